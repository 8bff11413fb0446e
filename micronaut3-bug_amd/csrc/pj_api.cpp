// pj_api.cpp — the C ABI of libpetjson (include/petjson.h).
//
// A context owns one HIP stream on one gfx950 device plus growable device
// scratch (look-back words, decode index arrays, host-path staging).  Every
// entry point validates its arguments on the host (shapes the kernels and
// their grids assume) before launching anything, synchronises its stream
// before returning, and reports failures as pj_status plus pj_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <string>
#include <thread>
#include <vector>

#include "petjson.h"
#include "pj_host_lock.h"
#include "pj_kernels.h"

namespace {

thread_local std::string g_err;

pj_status fail(pj_status s, const std::string &msg) {
    g_err = msg;
    return s;
}

#define PJ_HIP(call)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(e_ == hipErrorOutOfMemory ? PJ_ERR_OUT_OF_MEMORY : PJ_ERR_DEVICE, \
                        std::string(#call) + ": " + hipGetErrorString(e_));              \
    } while (0)

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    hipError_t ensure(size_t want) {
        if (want <= n) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        size_t sz = std::max<size_t>(want + want / 8, 4096);
        hipError_t e = hipMalloc(&p, sz);
        if (e == hipSuccess) n = sz;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

constexpr int MAX_EV = 12;

// A copy engine between pageable host memory and the device: its own copy
// stream, two pinned bounce buffers and their events.
struct Xfer {
    hipStream_t s = nullptr;
    uint8_t *bounce[2] = {nullptr, nullptr};
    hipEvent_t bev[2] = {nullptr, nullptr};
    hipEvent_t done = nullptr;
    size_t chunk = 0;
};

inline uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

}  // namespace

struct pj_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    pj_options opt{PJ_INCLUDE_NON_EMPTY, 1, {PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT,
                                                 PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT, PJ_INCLUDE_DEFAULT}};
    DevBuf scan;        // tickets, totals, look-back words
    DevBuf index;       // decode: special bitmap, bad flags, line starts
    DevBuf stage_in;    // host path: input staging
    DevBuf stage_out;   // host path: output staging
    DevBuf stage_out2;  // streamed host decode: the other segment's output staging
    DevBuf tape;        // decode: per-line results of the validating walk
    DevBuf seg_in[2];   // streamed host decode: input segments (double buffer)
    uint64_t *pinned = nullptr;   // 64 u64 of pinned host memory for results
    // host entry points: one copy engine per direction (made on first use),
    // so that a copy in and a copy out can run at once
    Xfer xin, xout;
    hipEvent_t seg_ready = nullptr;   // streamed decode: a segment's columns are final
    hipEvent_t seg_done[2] = {};      // streamed encode: a segment's bytes and length are final
    uint64_t *noalloc_scratch = nullptr;  // this device's fixed encode scratch (device address)
    bool flat_wide = false;       // flat encodes use the wide tile (records seen too long for the compact one)
    bool big_seen = true;         // the last nested encode listed large records (k_enc_big gets a full grid)
    hipEvent_t ev[MAX_EV] = {};
    int n_ev = 0;
    float timings[MAX_EV] = {};
    int n_timings = 0;
};

namespace {

pj_status bind(pj_ctx *c) {
    if (!c) return fail(PJ_ERR_INVALID_ARG, "null context");
    PJ_HIP(hipSetDevice(c->device));
    return PJ_OK;
}

pj_status mark(pj_ctx *c) {  // record the next timing event
    if (c->n_ev < MAX_EV) PJ_HIP(hipEventRecord(c->ev[c->n_ev++], c->stream));
    return PJ_OK;
}

pj_status finish_timing(pj_ctx *c) {
    c->n_timings = 0;
    if (c->n_ev >= 2) {
        PJ_HIP(hipEventSynchronize(c->ev[c->n_ev - 1]));
        float ms = 0;
        PJ_HIP(hipEventElapsedTime(&ms, c->ev[0], c->ev[c->n_ev - 1]));
        c->timings[c->n_timings++] = ms;
        for (int k = 1; k < c->n_ev && c->n_timings < MAX_EV; k++) {
            PJ_HIP(hipEventElapsedTime(&ms, c->ev[k - 1], c->ev[k]));
            c->timings[c->n_timings++] = ms;
        }
    }
    return PJ_OK;
}

// ---------------------------------------------------------------- host copies
// The host entry points move data between the caller's (pageable) memory and
// the device through two pinned bounce buffers of 64 MiB on a copy
// stream: while the DMA engine moves chunk i, host threads copy chunk i + 1
// into (or chunk i - 1 out of) the other buffer, so PCIe and the host copies
// overlap instead of the driver's staging path serialising them.
// (PETJSON_XFER_CHUNK overrides the size when a context first copies; tests
// use small odd sizes to cross many chunk boundaries.)
size_t xfer_chunk() {
    static const size_t v = [] {
        const char *e = std::getenv("PETJSON_XFER_CHUNK");
        const size_t x = e ? std::strtoull(e, nullptr, 10) : 0;
        return x >= 4096 ? x : (size_t)64 << 20;
    }();
    return v;
}

pj_status xfer_init(Xfer &x) {
    if (x.s) return PJ_OK;
    x.chunk = xfer_chunk();
    PJ_HIP(hipStreamCreateWithFlags(&x.s, hipStreamNonBlocking));
    for (int b = 0; b < 2; b++) {
        PJ_HIP(hipHostMalloc((void **)&x.bounce[b], x.chunk, hipHostMallocDefault));
        PJ_HIP(hipEventCreateWithFlags(&x.bev[b], hipEventDisableTiming));
    }
    PJ_HIP(hipEventCreateWithFlags(&x.done, hipEventDisableTiming));
    return PJ_OK;
}
void xfer_free(Xfer &x) {
    if (x.s) (void)hipStreamSynchronize(x.s);
    for (int b = 0; b < 2; b++) {
        if (x.bounce[b]) (void)hipHostFree(x.bounce[b]);
        if (x.bev[b]) (void)hipEventDestroy(x.bev[b]);
    }
    if (x.done) (void)hipEventDestroy(x.done);
    if (x.s) (void)hipStreamDestroy(x.s);
    x = Xfer{};
}

// n bytes from s to d on up to 16 host threads (at least 4 MiB each).
void par_copy(void *d, const void *s, size_t n) {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t T = std::min<size_t>({(size_t)std::min(hw, 16u), n / (4u << 20) + 1});
    if (T <= 1) {
        std::memcpy(d, s, n);
        return;
    }
    const size_t per = ((n + T - 1) / T + 4095) & ~size_t(4095);
    std::vector<std::thread> th;
    for (size_t k = 1; k < T && k * per < n; k++)
        th.emplace_back([=] { std::memcpy(static_cast<uint8_t *>(d) + k * per, static_cast<const uint8_t *>(s) + k * per,
                                          std::min(per, n - k * per)); });
    std::memcpy(d, s, std::min(per, n));
    for (auto &x : th) x.join();
}

// Whether host bytes [p, p + n) are pinned memory (pj_host_alloc, or any
// hipHostMalloc): such bytes move by DMA straight from / to the caller's
// buffer, with no copy through the bounce buffers.
bool pinned_host(const void *p, size_t n) {
    for (const void *q : {p, static_cast<const void *>(static_cast<const uint8_t *>(p) + n - 1)}) {
        hipPointerAttribute_t a;
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        if (a.type != hipMemoryTypeHost) return false;
    }
    return true;
}

// Host -> device; returns when the data is on the device.  With order_stream
// the context stream also waits for it before its next work; a second host
// thread copying while the context stream runs passes false, so that the
// work the main thread is queueing meanwhile does not wait for its copy.
// With wait false a copy from pinned memory is only queued: h2d_wait then
// waits for every copy queued so far, so that the slices of a column set
// cost one wait, not one each.
pj_status h2d_wait(pj_ctx *c, bool order_stream = true) {
    Xfer &x = c->xin;
    pj_status s = xfer_init(x);
    if (s) return s;
    PJ_HIP(hipEventRecord(x.done, x.s));
    if (order_stream) PJ_HIP(hipStreamWaitEvent(c->stream, x.done, 0));
    PJ_HIP(hipEventSynchronize(x.done));
    return PJ_OK;
}
pj_status h2d(pj_ctx *c, void *dev, const void *host, size_t n, bool order_stream = true, bool wait = true) {
    if (!n) return PJ_OK;
    Xfer &x = c->xin;
    pj_status s = xfer_init(x);
    if (s) return s;
    if (pinned_host(host, n)) {
        PJ_HIP(hipMemcpyAsync(dev, host, n, hipMemcpyHostToDevice, x.s));
        if (!wait) return PJ_OK;
    } else for (size_t off = 0, i = 0; off < n; off += x.chunk, i++) {
        const size_t k = std::min(x.chunk, n - off);
        const int b = (int)(i & 1);
        if (i >= 2) PJ_HIP(hipEventSynchronize(x.bev[b]));      // the DMA that last read this buffer is done
        par_copy(x.bounce[b], static_cast<const uint8_t *>(host) + off, k);
        PJ_HIP(hipMemcpyAsync(static_cast<uint8_t *>(dev) + off, x.bounce[b], k, hipMemcpyHostToDevice, x.s));
        PJ_HIP(hipEventRecord(x.bev[b], x.s));
    }
    PJ_HIP(hipEventRecord(x.done, x.s));
    if (order_stream) PJ_HIP(hipStreamWaitEvent(c->stream, x.done, 0));
    // the bounce buffers are reused by the next copy: wait for the last DMAs
    PJ_HIP(hipEventSynchronize(x.done));
    return PJ_OK;
}

// Device -> host, after the work the event `after` marks (by default the
// context stream's work so far); returns when the bytes are in host memory.
// With wait false a copy into pinned memory is only queued: d2h_wait then
// waits for every copy queued so far.
pj_status d2h_wait(pj_ctx *c) {
    Xfer &x = c->xout;
    pj_status s = xfer_init(x);
    if (s) return s;
    PJ_HIP(hipEventRecord(x.bev[0], x.s));
    PJ_HIP(hipEventSynchronize(x.bev[0]));
    return PJ_OK;
}
pj_status d2h(pj_ctx *c, void *host, const void *dev, size_t n, hipEvent_t after = nullptr, bool wait = true) {
    if (!n) return PJ_OK;
    Xfer &x = c->xout;
    pj_status s = xfer_init(x);
    if (s) return s;
    if (!after) {
        PJ_HIP(hipEventRecord(x.done, c->stream));
        after = x.done;
    }
    PJ_HIP(hipStreamWaitEvent(x.s, after, 0));
    if (pinned_host(host, n)) {
        PJ_HIP(hipMemcpyAsync(host, dev, n, hipMemcpyDeviceToHost, x.s));
        return wait ? d2h_wait(c) : PJ_OK;
    }
    const size_t chunks = (n + x.chunk - 1) / x.chunk;
    auto issue = [&](size_t i) -> pj_status {
        const size_t off = i * x.chunk, k = std::min(x.chunk, n - off);
        PJ_HIP(hipMemcpyAsync(x.bounce[i & 1], static_cast<const uint8_t *>(dev) + off, k, hipMemcpyDeviceToHost, x.s));
        PJ_HIP(hipEventRecord(x.bev[i & 1], x.s));
        return PJ_OK;
    };
    if ((s = issue(0))) return s;
    for (size_t i = 0; i < chunks; i++) {
        // the other buffer's host copy (chunk i - 1) is done: start chunk i + 1's DMA into it
        if (i + 1 < chunks && (s = issue(i + 1))) return s;
        PJ_HIP(hipEventSynchronize(x.bev[i & 1]));
        const size_t off = i * x.chunk;
        par_copy(static_cast<uint8_t *>(host) + off, x.bounce[i & 1], std::min(x.chunk, n - off));
    }
    return PJ_OK;
}

bool nested_cols(const pj_pet_columns *c) { return c->cat_id || c->photo_off || c->tag_off; }
uint64_t enc_big_cap() {
    if (const char *e = std::getenv("PETJSON_ENC_BIG_CAP")) return std::strtoull(e, nullptr, 10);
    return 1ull << 20;
}
// PETJSON_ENC_TWO_PASS=1 writes nested records at the offsets of the
// measuring pass instead of with the single pass (kept to compare the two).
bool enc_two_pass() {
    const char *e = std::getenv("PETJSON_ENC_TWO_PASS");
    return e && e[0] == '1';
}

pj_status check_enc_cols(const pj_pet_columns *c) {
    if (c->n_pets == 0) return PJ_OK;
    if (!c->name_off || !c->name_bytes) return fail(PJ_ERR_INVALID_ARG, "name_off / name_bytes required");
    if (!c->id && (!c->flags)) return fail(PJ_ERR_INVALID_ARG, "id column NULL requires a flags column");
    if (c->cat_id && (!c->cat_name_off || !c->cat_name_bytes))
        return fail(PJ_ERR_INVALID_ARG, "category group incomplete");
    if (c->photo_off && (!c->url_off || !c->url_bytes)) return fail(PJ_ERR_INVALID_ARG, "photoUrls group incomplete");
    if (c->tag_off && (!c->tag_id || !c->tag_name_off || !c->tag_name_bytes))
        return fail(PJ_ERR_INVALID_ARG, "tags group incomplete");
    if (c->n_pets > (1ull << 40)) return fail(PJ_ERR_INVALID_ARG, "too many records");
    return PJ_OK;
}

// Look-back wait bound for launch-ordered blocks: 200 ms of the 100 MHz wall
// clock, or PETJSON_SPIN_LIMIT_TICKS (tests force the redo path with a tiny
// bound).
// Whether the decode keeps a line tape (PETJSON_DECODE_TAPE=0 turns it off;
// tests cover both paths).
bool decode_tape_enabled() {
    const char *e = std::getenv("PETJSON_DECODE_TAPE");
    return !e || std::strtoull(e, nullptr, 10) != 0;
}

uint64_t spin_limit() {
    if (const char *e = std::getenv("PETJSON_SPIN_LIMIT_TICKS")) {
        const unsigned long long v = std::strtoull(e, nullptr, 10);
        if (v) return v;
    }
    return 20000000;
}

// The context's options as the encode kernels read them.
void set_enc_options(const pj_ctx *ctx, EncParams &P) {
    for (int k = 0; k < PJ_FIELD_COUNT; k++) {
        const int32_t m = ctx->opt.field_inclusion[k];
        P.incl[k] = (uint8_t)(m == PJ_INCLUDE_DEFAULT ? ctx->opt.inclusion : m);
    }
    P.hexa = ctx->opt.hex_upper ? 'A' : 'a';
}

bool format_ok(int f) { return f == PJ_FORMAT_ARRAY || f == PJ_FORMAT_NDJSON || f == PJ_FORMAT_PRETTY; }

// One segment of a streamed host encode (compact formats): the local index
// of the input's first and last record (or ~0 when the segment holds
// neither), and the pinned word that receives the segment's length before
// the event is recorded.  encode_impl then returns as soon as the work is
// queued.
struct EncSeg {
    uint64_t first, last;
    uint64_t *len;
    hipEvent_t done;
};

// fixed_scratch: encode into the device's fixed scratch array instead of
// the context's growable buffer (pj_encode_device_noalloc); nothing is
// allocated on that path.
pj_status encode_impl(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint8_t *out, uint64_t cap,
                      uint64_t *out_len, bool count_only, bool fixed_scratch = false, const EncSeg *seg = nullptr) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!format_ok(format)) return fail(PJ_ERR_INVALID_ARG, "bad format");
    if (!count_only && cap > 0 && !out) return fail(PJ_ERR_INVALID_ARG, "null output with capacity");
    if ((s = check_enc_cols(cols))) return s;
    ctx->n_ev = 0;
    const uint64_t n = cols->n_pets;
    if (n == 0) {
        // "[]", "[ ]" (pretty) or nothing
        const uint64_t len = format == PJ_FORMAT_ARRAY ? 2 : format == PJ_FORMAT_PRETTY ? 3 : 0;
        *out_len = len;
        if (!count_only && len && len <= cap) {
            if ((s = mark(ctx))) return s;
            const uint32_t w = format == PJ_FORMAT_ARRAY ? '[' | (']' << 8) : '[' | (' ' << 8) | (']' << 16);
            PJ_HIP(pj_launch_put_bytes(out, w, (int)len, ctx->stream));
            if ((s = mark(ctx))) return s;
        }
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        if ((s = finish_timing(ctx))) return s;
        return len > cap && !count_only ? fail(PJ_ERR_CAPACITY, "output capacity too small") : PJ_OK;
    }
    const bool pretty = format == PJ_FORMAT_PRETTY;
    // pretty nested records are written by the tiled encode; the size alone
    // comes faster from the one-thread-per-record kernel (1.6 against 2.55 ms
    // at 10M records), and the fixed scratch, sized for blocks of 96, keeps
    // that kernel too
    const bool pretty_tiled = pretty && nested_cols(cols) && !fixed_scratch && !count_only;
    const uint64_t bt = (uint64_t)(pretty_tiled ? pj_encode_pretty_tile_records()
                                   : pretty     ? pj_encode_pretty_records()
                                                : pj_encode_block_records(nested_cols(cols)));
    const uint64_t nblk = (n + bt - 1) / bt;
    // Nested records: the size alone comes from the measuring pass
    // (k_enc_measure), which also gives every block its bounds and offset.
    // The bytes come from the single pass, each block placed by its own
    // look-back; it measured faster than the measuring pass followed by a
    // writer at the given offsets (PETJSON_ENC_TWO_PASS=1).  The fixed
    // scratch of the no-allocation entry point holds only the single pass.
    const bool two_pass = !pretty && nested_cols(cols) && !fixed_scratch && !seg && (count_only || enc_two_pass());
    // Nested records too large for the tile path (long names or lists) are
    // written after the pass by k_enc_big, up to 2^20 of them per call (the
    // rest by the pass itself; PETJSON_ENC_BIG_CAP sets another limit, 0 for
    // none); the fixed scratch holds no such list.
    const bool defer_big = nested_cols(cols) && !pretty && !count_only && !fixed_scratch;
    const uint64_t big_cap = defer_big ? std::min<uint64_t>(n, enc_big_cap()) : 0;
    uint64_t *sc;
    std::unique_lock<std::mutex> noalloc_guard;
    if (fixed_scratch) {
        if (n > PJ_NOALLOC_MAX_RECORDS(nested_cols(cols)) || nblk + 4 + 128 > PJ_NOALLOC_SCRATCH_WORDS)
            return fail(PJ_ERR_INVALID_ARG, "pj_encode_device_noalloc: " + std::to_string(n) +
                                                " records exceed the fixed scratch (at most " +
                                                std::to_string(PJ_NOALLOC_MAX_RECORDS(nested_cols(cols))) + ")");
        sc = ctx->noalloc_scratch;
        // every call on this GPU shares the array: one call at a time, until
        // its stream has drained (the lock is released when this returns)
        noalloc_guard = std::unique_lock<std::mutex>(pj::noalloc_lock(ctx->device));
    } else {
        PJ_HIP(ctx->scan.ensure((nblk + 4 + 128 + (two_pass ? GEO_WORDS * nblk : 0) + 2 * big_cap) * sizeof(uint64_t)));
        sc = static_cast<uint64_t *>(ctx->scan.p);
    }
    EncParams P;
    std::memset(&P, 0, sizeof P);
    P.c = *cols;
    P.n = n;
    P.first = seg ? seg->first : 0;
    P.last = seg ? seg->last : n - 1;
    P.format = format;
    set_enc_options(ctx, P);
    P.count_only = count_only ? 1 : 0;
    P.out = out;
    P.cap = count_only ? 0 : cap;
    // scan buffer: ticket, total, fallback-block count, large-record count,
    // look-back words (these zeroed before each pass), dummy, block
    // geometry (two passes), large-record list
    P.ticket = reinterpret_cast<unsigned long long *>(sc);
    P.total = sc + 1;
    P.nfall = reinterpret_cast<unsigned long long *>(sc + 2);
    P.big_count = reinterpret_cast<unsigned long long *>(sc + 3);
    P.state = sc + 4;
    P.dummy = reinterpret_cast<uint32_t *>(sc + 4 + nblk);   // 128 u64 = PJ_BLOCK dwords
    uint64_t *geo = two_pass ? sc + 4 + nblk + 128 : nullptr;
    P.big_list = sc + 4 + nblk + 128 + (two_pass ? GEO_WORDS * nblk : 0);
    P.big_cap = big_cap;
    // Nested records run on persistent workgroups that claim their blocks by
    // ticket.  Flat blocks run one per workgroup in launch order (no ticket
    // atomic on the critical path) with bounded look-back waits: should a
    // block wait past the bound (a predecessor not yet running), it flags
    // the launch, which is then redone with ticket-ordered blocks.
    P.order_by_id = nested_cols(cols) || pretty || seg ? 0 : 1;
    P.spin_limit = spin_limit();
    for (int attempt = 0;; attempt++) {
        if ((s = mark(ctx))) return s;
        PJ_HIP(pj_launch_fill_u64(sc, nblk + 4, 0, ctx->stream));
        if ((s = mark(ctx))) return s;
        if (pretty_tiled) PJ_HIP(pj_launch_encode_pretty(P, ctx->stream));
        else if (pretty) PJ_HIP(pj_launch_encode_rows(P, true, ctx->stream));
        else if (two_pass) {
            P.geo = geo;
            PJ_HIP(pj_launch_encode_measure(P, ctx->stream));
            if (!count_only) {
                if ((s = mark(ctx))) return s;
                PJ_HIP(pj_launch_fill_u64(sc, 1, 0, ctx->stream));   // the writer's tickets
                P.geo = geo;
                PJ_HIP(pj_launch_encode(P, true, false, ctx->stream));
                if (big_cap) PJ_HIP(pj_launch_encode_big(P, ctx->big_seen, ctx->stream));
            }
        } else {
            PJ_HIP(pj_launch_encode(P, nested_cols(cols), ctx->flat_wide, ctx->stream));
            if (big_cap) PJ_HIP(pj_launch_encode_big(P, ctx->big_seen, ctx->stream));
        }
        if ((s = mark(ctx))) return s;
        if (seg) {
            PJ_HIP(hipMemcpyAsync(seg->len, sc + 1, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
            PJ_HIP(hipEventRecord(seg->done, ctx->stream));
            return PJ_OK;
        }
        PJ_HIP(hipMemcpyAsync(ctx->pinned, sc, 4 * sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        if (!P.order_by_id || ctx->pinned[0] == 0 || attempt > 0) break;
        P.order_by_id = 0;                                      // redo in ticket order
        ctx->n_ev = 0;
    }
    // the next nested encode's k_enc_big grid follows this one's large records
    if (big_cap) ctx->big_seen = ctx->pinned[3] != 0;
    // flat records too long for the compact tile: later calls use the wide one
    if (!pretty && !nested_cols(cols) && !ctx->flat_wide && ctx->pinned[2] * 64 > nblk) ctx->flat_wide = true;
    if ((s = finish_timing(ctx))) return s;
    *out_len = ctx->pinned[1];
    if (!count_only && *out_len > cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    return PJ_OK;
}

// ---------------------------------------------------------- host staging
struct Layout {  // byte offsets of each column inside one staging buffer
    uint64_t off[17];
    uint64_t size[17];
    uint64_t total;
};

// Column sizes implied by a host column set (offset arrays give the counts).
void host_layout(const pj_pet_columns *c, Layout *L) {
    const uint64_t n = c->n_pets;
    uint64_t nu = c->photo_off ? c->photo_off[n] : 0, nt = c->tag_off ? c->tag_off[n] : 0;
    uint64_t sz[17] = {
        c->id ? n * 8 : 0,
        c->flags ? n : 0,
        c->status ? n : 0,
        c->name_off ? (n + 1) * 8 : 0,
        c->name_bytes ? c->name_off[n] : 0,
        c->cat_id ? n * 8 : 0,
        c->cat_flags ? n : 0,
        c->cat_name_off ? (n + 1) * 8 : 0,
        c->cat_name_bytes ? c->cat_name_off[n] : 0,
        c->photo_off ? (n + 1) * 8 : 0,
        c->url_off ? (nu + 1) * 8 : 0,
        c->url_bytes ? c->url_off[nu] : 0,
        c->tag_off ? (n + 1) * 8 : 0,
        c->tag_id ? nt * 8 : 0,
        c->tag_flags ? nt : 0,
        c->tag_name_off ? (nt + 1) * 8 : 0,
        c->tag_name_bytes ? c->tag_name_off[nt] : 0,
    };
    uint64_t o = 0;
    for (int k = 0; k < 17; k++) {
        L->off[k] = o;
        L->size[k] = sz[k];
        o += align256(sz[k] + 4);  // +4: aligned-dword reads may touch the tail
    }
    L->total = o;
}

void **col_ptrs(pj_pet_columns *c, void **v) {
    void *src[17] = {c->id, c->flags, c->status, c->name_off, c->name_bytes, c->cat_id, c->cat_flags,
                     c->cat_name_off, c->cat_name_bytes, c->photo_off, c->url_off, c->url_bytes,
                     c->tag_off, c->tag_id, c->tag_flags, c->tag_name_off, c->tag_name_bytes};
    std::memcpy(v, src, sizeof src);
    return v;
}

void set_col_ptrs(pj_pet_columns *c, void *const *v) {
    c->id = (int64_t *)v[0]; c->flags = (uint8_t *)v[1]; c->status = (uint8_t *)v[2];
    c->name_off = (uint64_t *)v[3]; c->name_bytes = (uint8_t *)v[4]; c->cat_id = (int64_t *)v[5];
    c->cat_flags = (uint8_t *)v[6]; c->cat_name_off = (uint64_t *)v[7]; c->cat_name_bytes = (uint8_t *)v[8];
    c->photo_off = (uint64_t *)v[9]; c->url_off = (uint64_t *)v[10]; c->url_bytes = (uint8_t *)v[11];
    c->tag_off = (uint64_t *)v[12]; c->tag_id = (int64_t *)v[13]; c->tag_flags = (uint8_t *)v[14];
    c->tag_name_off = (uint64_t *)v[15]; c->tag_name_bytes = (uint8_t *)v[16];
}

}  // namespace

// ===================================================================== ABI
extern "C" {

const char *pj_last_error(void) { return g_err.c_str(); }

void pj_default_options(pj_options *o) {
    if (!o) return;
    o->inclusion = PJ_INCLUDE_NON_EMPTY;
    o->hex_upper = 1;
    for (int k = 0; k < PJ_FIELD_COUNT; k++) o->field_inclusion[k] = PJ_INCLUDE_DEFAULT;
}

pj_ctx *pj_create(int device, pj_status *status) {
    auto set = [&](pj_status s) { if (status) *status = s; };
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        g_err = "no HIP device";
        set(PJ_ERR_NO_DEVICE);
        return nullptr;
    }
    if (device < 0 || device >= n) {
        g_err = "device index out of range";
        set(PJ_ERR_INVALID_ARG);
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess || std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_err = std::string("libpetjson is built for gfx950; device is ") + prop.gcnArchName;
        set(PJ_ERR_NO_DEVICE);
        return nullptr;
    }
    pj_ctx *c = new pj_ctx();
    c->device = device;
    bool ok = hipSetDevice(device) == hipSuccess && hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) == hipSuccess &&
              hipHostMalloc((void **)&c->pinned, 64 * sizeof(uint64_t), hipHostMallocDefault) == hipSuccess &&
              pj_noalloc_scratch_init(device, &c->noalloc_scratch) == hipSuccess;
    for (int k = 0; ok && k < MAX_EV; k++) ok = hipEventCreate(&c->ev[k]) == hipSuccess;
    if (!ok) {
        g_err = "context set-up failed";
        pj_destroy(c);
        set(PJ_ERR_DEVICE);
        return nullptr;
    }
    set(PJ_OK);
    return c;
}

void pj_destroy(pj_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    c->scan.release();
    c->index.release();
    c->stage_in.release();
    c->stage_out.release();
    c->stage_out2.release();
    c->tape.release();
    c->seg_in[0].release();
    c->seg_in[1].release();
    for (auto &e : c->ev) if (e) (void)hipEventDestroy(e);
    if (c->pinned) (void)hipHostFree(c->pinned);
    xfer_free(c->xin);
    xfer_free(c->xout);
    if (c->seg_ready) (void)hipEventDestroy(c->seg_ready);
    for (hipEvent_t e : c->seg_done)
        if (e) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

pj_status pj_set_options(pj_ctx *c, const pj_options *o) {
    if (!c || !o) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (o->inclusion < PJ_INCLUDE_NON_EMPTY || o->inclusion > PJ_INCLUDE_ALWAYS)
        return fail(PJ_ERR_INVALID_ARG, "bad inclusion mode");
    for (int k = 0; k < PJ_FIELD_COUNT; k++)
        if (o->field_inclusion[k] != PJ_INCLUDE_DEFAULT &&
            (o->field_inclusion[k] < PJ_INCLUDE_NON_EMPTY || o->field_inclusion[k] > PJ_INCLUDE_ALWAYS))
            return fail(PJ_ERR_INVALID_ARG, "bad inclusion mode for field " + std::to_string(k));
    c->opt = *o;
    c->opt.hex_upper = o->hex_upper ? 1 : 0;
    return PJ_OK;
}

int pj_last_timings(const pj_ctx *c, float *ms, int cap) {
    if (!c || !ms) return 0;
    int k = std::min(cap, c->n_timings);
    for (int i = 0; i < k; i++) ms[i] = c->timings[i];
    return k;
}

pj_status pj_encode_by_status_device(pj_ctx *ctx, const pj_pet_columns *cols, uint32_t status_mask, int format,
                                     uint8_t *out, uint64_t out_cap, uint64_t *out_len, uint64_t *n_selected) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!format_ok(format)) return fail(PJ_ERR_INVALID_ARG, "bad format");
    if (status_mask & ~0xFu) return fail(PJ_ERR_INVALID_ARG, "status mask has bits past 3");
    if (out_cap > 0 && !out) return fail(PJ_ERR_INVALID_ARG, "null output with capacity");
    if ((s = check_enc_cols(cols))) return s;
    ctx->n_ev = 0;
    const uint64_t n = cols->n_pets, bt = (uint64_t)pj_encode_pretty_records(), nblk = (n + bt - 1) / bt;
    // scan buffer: selection (ticket, count, look-back words), encode
    // (ticket, total, look-back words), the selected indices
    const uint64_t w_sel = 2 + pj_select_blocks(n), w_enc = 2 + nblk;
    PJ_HIP(ctx->scan.ensure((w_sel + w_enc + n + 1) * sizeof(uint64_t)));
    uint64_t *sc = static_cast<uint64_t *>(ctx->scan.p), *ec = sc + w_sel, *sel = ec + w_enc;
    EncParams P;
    std::memset(&P, 0, sizeof P);
    P.c = *cols;
    P.format = format;
    set_enc_options(ctx, P);
    P.out = out;
    P.cap = out_cap;
    uint64_t m = 0;
    if (n) {
        P.ticket = reinterpret_cast<unsigned long long *>(sc);
        P.total = sc + 1;
        P.state = sc + 2;
        if ((s = mark(ctx))) return s;
        PJ_HIP(pj_launch_fill_u64(sc, w_sel + w_enc, 0, ctx->stream));
        if ((s = mark(ctx))) return s;
        PJ_HIP(pj_launch_select_status(P, status_mask, sel, ctx->stream));
        if ((s = mark(ctx))) return s;
        PJ_HIP(hipMemcpyAsync(ctx->pinned, sc + 1, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        m = ctx->pinned[0];
    }
    if (n_selected) *n_selected = m;
    if (m == 0) {
        // "[]", "[ ]" (pretty) or nothing
        const uint64_t len = format == PJ_FORMAT_ARRAY ? 2 : format == PJ_FORMAT_PRETTY ? 3 : 0;
        *out_len = len;
        if (len && len <= out_cap) {
            const uint32_t w = format == PJ_FORMAT_ARRAY ? '[' | (']' << 8) : '[' | (' ' << 8) | (']' << 16);
            PJ_HIP(pj_launch_put_bytes(out, w, (int)len, ctx->stream));
        }
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        if ((s = finish_timing(ctx))) return s;
        return len > out_cap ? fail(PJ_ERR_CAPACITY, "output capacity too small") : PJ_OK;
    }
    P.n = m;
    P.first = 0;
    P.last = m - 1;
    P.sel = sel;
    P.ticket = reinterpret_cast<unsigned long long *>(ec);
    P.total = ec + 1;
    P.state = ec + 2;
    PJ_HIP(pj_launch_encode_rows(P, format == PJ_FORMAT_PRETTY, ctx->stream));
    if ((s = mark(ctx))) return s;
    PJ_HIP(hipMemcpyAsync(ctx->pinned, ec + 1, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
    PJ_HIP(hipStreamSynchronize(ctx->stream));
    if ((s = finish_timing(ctx))) return s;
    *out_len = ctx->pinned[0];
    if (*out_len > out_cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    return PJ_OK;
}

pj_status pj_encode_device(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint8_t *out, uint64_t out_cap,
                           uint64_t *out_len) {
    return encode_impl(ctx, cols, format, out, out_cap, out_len, false);
}

pj_status pj_encode_device_noalloc(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint8_t *out,
                                   uint64_t out_cap, uint64_t *out_len) {
    return encode_impl(ctx, cols, format, out, out_cap, out_len, false, true);
}

pj_status pj_encode_size_device(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint64_t *out_len) {
    return encode_impl(ctx, cols, format, nullptr, 0, out_len, true);
}

}  // extern "C"

namespace {
// Host Pet columns copied into the context's input staging buffer; *dc
// receives the same column set with device pointers.
pj_status stage_pet_cols(pj_ctx *ctx, const pj_pet_columns *cols, pj_pet_columns *dc) {
    pj_status s;
    Layout L;
    host_layout(cols, &L);
    PJ_HIP(ctx->stage_in.ensure(L.total));
    uint8_t *base = static_cast<uint8_t *>(ctx->stage_in.p);
    void *hp[17], *dp[17];
    pj_pet_columns hc = *cols;
    *dc = *cols;
    col_ptrs(&hc, hp);
    for (int k = 0; k < 17; k++) {
        dp[k] = hp[k] ? base + L.off[k] : nullptr;
        if (hp[k] && L.size[k] && (s = h2d(ctx, dp[k], hp[k], L.size[k], true, false))) return s;
    }
    if ((s = h2d_wait(ctx))) return s;
    set_col_ptrs(dc, dp);
    return PJ_OK;
}
// ---- streamed host encode
// pj_encode_host of an input over 512 MiB of columns (compact formats) runs
// in segments of records of about 256 MiB (PETJSON_ENCODE_SEGMENT sets the
// size, and then anything over it streams; on the 0.35 GB flat benchmark
// input, segments of 44 MB measured slower than one piece).
// While segment k encodes on the context stream, a host thread copies
// segment k + 1's column slices in (engine xin), and segment k - 1's bytes go
// out (engine xout) to the caller's buffer at the running offset; PCIe is
// full duplex, so the two copies run at once.  A segment's slices keep the
// column layout: offsets stay absolute, and a slice indexed by them gets a
// device pointer shifted back by its first offset.  Byte slices sit at the
// address their first byte has in the input, modulo 16, with 16 bytes on
// either side (the staging loads read aligned 16-byte chunks around them).
uint64_t enc_segment_bytes() {
    if (const char *e = std::getenv("PETJSON_ENCODE_SEGMENT")) {
        const unsigned long long v = std::strtoull(e, nullptr, 10);
        if (v) return v;
    }
    return 256ull << 20;
}
uint64_t enc_stream_above() {
    if (std::getenv("PETJSON_ENCODE_SEGMENT")) return enc_segment_bytes();
    return 2 * enc_segment_bytes();
}

// The column slices of records [r0, r1): per column (col_ptrs order) its
// first byte in the host column, its size, its offset in the device buffer
// and the shift of the device pointer.
struct EncSlices {
    uint64_t src[17], size[17], off[17], shift[17];
    uint64_t total;
};
void enc_slices(const pj_pet_columns *c, uint64_t r0, uint64_t r1, EncSlices *E) {
    const uint64_t m = r1 - r0;
    const uint64_t u0 = c->photo_off ? c->photo_off[r0] : 0, u1 = c->photo_off ? c->photo_off[r1] : 0;
    const uint64_t t0 = c->tag_off ? c->tag_off[r0] : 0, t1 = c->tag_off ? c->tag_off[r1] : 0;
    void *hp[17];
    pj_pet_columns hc = *c;
    col_ptrs(&hc, hp);
    // byte ranges of the string columns: [first byte, end)
    const uint64_t nb0 = c->name_off[r0], nb1 = c->name_off[r1];
    const uint64_t cb0 = c->cat_name_off ? c->cat_name_off[r0] : 0, cb1 = c->cat_name_off ? c->cat_name_off[r1] : 0;
    const uint64_t ub0 = c->photo_off ? c->url_off[u0] : 0, ub1 = c->photo_off ? c->url_off[u1] : 0;
    const uint64_t gb0 = c->tag_off ? c->tag_name_off[t0] : 0, gb1 = c->tag_off ? c->tag_name_off[t1] : 0;
    const uint64_t src[17] = {r0 * 8, r0, r0, r0 * 8, nb0, r0 * 8, r0, r0 * 8, cb0,
                              r0 * 8, u0 * 8, ub0, r0 * 8, t0 * 8, t0, t0 * 8, gb0};
    const uint64_t size[17] = {m * 8, m, m, (m + 1) * 8, nb1 - nb0, m * 8, m, (m + 1) * 8, cb1 - cb0,
                               (m + 1) * 8, (u1 - u0 + 1) * 8, ub1 - ub0, (m + 1) * 8, (t1 - t0) * 8, t1 - t0,
                               (t1 - t0 + 1) * 8, gb1 - gb0};
    // the columns indexed by item or byte offsets: the pointer moves back by
    // the slice's first index (record columns are indexed from the segment's
    // first record)
    const uint64_t shift[17] = {0, 0, 0, 0, nb0, 0, 0, 0, cb0, 0, u0 * 8, ub0, 0, t0 * 8, t0, t0 * 8, gb0};
    uint64_t o = 0;
    for (int k = 0; k < 17; k++) {
        const bool on = hp[k] != nullptr;
        E->src[k] = src[k];
        E->size[k] = on ? size[k] : 0;
        E->shift[k] = shift[k];
        o = align256(o) + 16;
        o += (src[k] - o) & 15;                 // the same address mod 16 as in the input
        E->off[k] = o;
        o += E->size[k] + 16;
    }
    E->total = align256(o);
}

// Records [r0, r1) of host columns as a column set of their own (for
// pj_encode_bound): record columns start at r0; offsets stay absolute.
pj_pet_columns seg_view(const pj_pet_columns *c, uint64_t r0, uint64_t r1) {
    pj_pet_columns v = *c;
    v.n_pets = r1 - r0;
    if (v.id) v.id += r0;
    if (v.flags) v.flags += r0;
    if (v.status) v.status += r0;
    v.name_off += r0;
    if (v.cat_id) v.cat_id += r0;
    if (v.cat_flags) v.cat_flags += r0;
    if (v.cat_name_off) v.cat_name_off += r0;
    if (v.photo_off) v.photo_off += r0;
    if (v.tag_off) v.tag_off += r0;
    return v;
}

pj_status encode_host_stream(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint8_t *out, uint64_t cap,
                             uint64_t *out_len) {
    const uint64_t n = cols->n_pets;
    Layout L;
    host_layout(cols, &L);
    const uint64_t seg = enc_segment_bytes();
    const uint64_t nseg = std::max<uint64_t>(2, (L.total + seg - 1) / seg);
    const uint64_t S = (n + nseg - 1) / nseg;
    // buffers sized once for the largest segment: its slices, and its
    // output (pj_encode_bound of its records)
    uint64_t in_max = 0, out_max = 0;
    for (uint64_t r0 = 0; r0 < n; r0 += S) {
        const uint64_t r1 = std::min(n, r0 + S);
        EncSlices E;
        enc_slices(cols, r0, r1, &E);
        pj_pet_columns hv = seg_view(cols, r0, r1);
        uint64_t bound = 0;
        pj_status s0 = pj_encode_bound(&hv, format, &bound);
        if (s0) return s0;
        in_max = std::max(in_max, E.total);
        out_max = std::max(out_max, bound + 64);
    }
    DevBuf *stage[2] = {&ctx->stage_out, &ctx->stage_out2};
    for (int k = 0; k < 2; k++) {
        PJ_HIP(ctx->seg_in[k].ensure(in_max));
        PJ_HIP(stage[k]->ensure(out_max));
        if (!ctx->seg_done[k]) PJ_HIP(hipEventCreateWithFlags(&ctx->seg_done[k], hipEventDisableTiming));
    }
    struct Job {
        std::thread th;
        pj_status st = PJ_OK;
        std::string err;
        pj_status join() {
            if (th.joinable()) th.join();
            const pj_status r = st;
            st = PJ_OK;
            return r;
        }
    };
    Job cin, cout;
    auto finish = [&](pj_status r) -> pj_status {
        const pj_status a1 = cin.join(), a2 = cout.join();
        if (r) return r;
        if (a1) return fail(a1, cin.err);
        if (a2) return fail(a2, cout.err);
        return PJ_OK;
    };
    // the slices of records [r0, r1) into slot k's input buffer
    auto load = [&](int k, uint64_t r0, uint64_t r1) -> pj_status {
        EncSlices E;
        enc_slices(cols, r0, r1, &E);
        void *hp[17];
        pj_pet_columns hc = *cols;
        col_ptrs(&hc, hp);
        uint8_t *D = static_cast<uint8_t *>(ctx->seg_in[k].p);
        for (int j = 0; j < 17; j++) {
            if (!E.size[j]) continue;
            const pj_status r =
                h2d(ctx, D + E.off[j], static_cast<const uint8_t *>(hp[j]) + E.src[j], E.size[j], false, false);
            if (r) return r;
        }
        return h2d_wait(ctx, false);
    };
    pj_status s = load(0, 0, std::min(n, S));
    if (s) return s;
    uint64_t done = 0;                        // bytes of the segments before this one
    int k = 0;
    for (uint64_t r0 = 0; r0 < n; r0 += S, k ^= 1) {
        const uint64_t r1 = std::min(n, r0 + S);
        // segment k is on the device: its columns, shifted as its slices say
        if (const pj_status c1 = cin.join()) return finish(fail(c1, cin.err));
        EncSlices E;
        enc_slices(cols, r0, r1, &E);
        void *dp[17];
        {
            void *hp[17];
            pj_pet_columns hc = *cols;
            col_ptrs(&hc, hp);
            const uintptr_t D = reinterpret_cast<uintptr_t>(ctx->seg_in[k].p);
            for (int j = 0; j < 17; j++) dp[j] = hp[j] ? reinterpret_cast<void *>(D + E.off[j] - E.shift[j]) : nullptr;
        }
        pj_pet_columns dc = *cols;
        set_col_ptrs(&dc, dp);
        dc.n_pets = r1 - r0;
        const EncSeg es{r0 == 0 ? 0 : ~0ull, r1 == n ? r1 - r0 - 1 : ~0ull, ctx->pinned + 48 + k, ctx->seg_done[k]};
        uint64_t unused = 0;
        if ((s = encode_impl(ctx, &dc, format, static_cast<uint8_t *>(stage[k]->p), out_max, &unused, false, false, &es)))
            return finish(s);
        // segment k + 1 in while k encodes (its slot's input was read by
        // segment k - 1, whose encode is done: its length was read below)
        if (r1 < n) {
            const uint64_t a2 = r1, b2 = std::min(n, r1 + S);
            const int k2 = k ^ 1;
            cin.th = std::thread([&, k2, a2, b2] {
                pj_status r = bind(ctx);               // (HIP's current device is per thread)
                if (!r) r = load(k2, a2, b2);
                if (r) cin.err = pj_last_error();
                cin.st = r;
            });
        }
        // segment k - 1's bytes are out, so its output slot is free again
        if (const pj_status c2 = cout.join()) return finish(fail(c2, cout.err));
        if (const hipError_t x = hipEventSynchronize(ctx->seg_done[k]))
            return finish(fail(PJ_ERR_DEVICE, std::string("encode segment: ") + hipGetErrorString(x)));
        const uint64_t len = ctx->pinned[48 + k];
        // as much of segment k as fits the caller's buffer
        const uint64_t w = done >= cap ? 0 : std::min(len, cap - done);
        if (w) {
            uint8_t *dst = out + done;
            const void *src = stage[k]->p;
            hipEvent_t ready = ctx->seg_done[k];     // (recorded again only after this thread is joined)
            cout.th = std::thread([&, dst, src, w, ready] {
                pj_status q = bind(ctx);
                if (!q) q = d2h(ctx, dst, src, w, ready);
                if (q) cout.err = pj_last_error();
                cout.st = q;
            });
        }
        done += len;
    }
    if ((s = finish(PJ_OK))) return s;
    *out_len = done;
    if (done > cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    return PJ_OK;
}

}  // namespace

extern "C" {

pj_status pj_encode_by_status_host(pj_ctx *ctx, const pj_pet_columns *cols, uint32_t status_mask, int format,
                                   uint8_t *out, uint64_t out_cap, uint64_t *out_len, uint64_t *n_selected) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if ((s = check_enc_cols(cols))) return s;
    pj_pet_columns dc;
    if ((s = stage_pet_cols(ctx, cols, &dc))) return s;
    uint64_t need = 0;
    s = pj_encode_by_status_device(ctx, &dc, status_mask, format, nullptr, 0, &need, n_selected);
    if (s != PJ_OK && s != PJ_ERR_CAPACITY) return s;
    *out_len = need;
    if (need > out_cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    if (need == 0) return PJ_OK;
    if (!out) return fail(PJ_ERR_INVALID_ARG, "null output");
    PJ_HIP(ctx->stage_out.ensure(need + 4));
    uint64_t got = 0;
    if ((s = pj_encode_by_status_device(ctx, &dc, status_mask, format, static_cast<uint8_t *>(ctx->stage_out.p), need,
                                        &got, n_selected)))
        return s;
    if ((s = d2h(ctx, out, ctx->stage_out.p, got))) return s;
    *out_len = got;
    return PJ_OK;
}

pj_status pj_encode_host(pj_ctx *ctx, const pj_pet_columns *cols, int format, uint8_t *out, uint64_t out_cap,
                         uint64_t *out_len) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (cols->n_pets && (s = check_enc_cols(cols))) return s;
    if (cols->n_pets && format != PJ_FORMAT_PRETTY) {
        if (!format_ok(format)) return fail(PJ_ERR_INVALID_ARG, "bad format");
        Layout L;
        host_layout(cols, &L);
        if (L.total > enc_stream_above()) {
            if (!out && out_cap) return fail(PJ_ERR_INVALID_ARG, "null output");
            return encode_host_stream(ctx, cols, format, out, out_cap, out_len);
        }
    }
    pj_pet_columns dc;
    if ((s = stage_pet_cols(ctx, cols, &dc))) return s;
    uint64_t need = 0;
    if ((s = pj_encode_size_device(ctx, &dc, format, &need))) return s;
    *out_len = need;
    if (need > out_cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    if (need == 0) return PJ_OK;
    if (!out) return fail(PJ_ERR_INVALID_ARG, "null output");
    PJ_HIP(ctx->stage_out.ensure(need + 4));
    uint64_t got = 0;
    if ((s = pj_encode_device(ctx, &dc, format, static_cast<uint8_t *>(ctx->stage_out.p), need, &got))) return s;
    if ((s = d2h(ctx, out, ctx->stage_out.p, got))) return s;
    *out_len = got;
    return PJ_OK;
}

pj_status pj_encode_bound(const pj_pet_columns *cols, int format, uint64_t *bound) {
    if (!cols || !bound) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!format_ok(format)) return fail(PJ_ERR_INVALID_ARG, "bad format");
    pj_status s;
    if ((s = check_enc_cols(cols))) return s;
    const uint64_t n = cols->n_pets;
    // per record: every Pet / Category property with a 20-character long,
    // the longest status and the framing; per url / tag item: its quotes,
    // separators and (tags) an object with both properties.  Pretty output
    // adds at most 64 bytes of whitespace per record, 1 per url and 32 per
    // tag.
    const bool pretty = format == PJ_FORMAT_PRETTY;
    uint64_t b = 3 + n * (pretty ? 320 : 256), str = 0;
    if (n) {
        str += cols->name_off[n] - cols->name_off[0];
        if (cols->cat_name_off) str += cols->cat_name_off[n] - cols->cat_name_off[0];
        if (cols->photo_off) {
            const uint64_t u0 = cols->photo_off[0], u1 = cols->photo_off[n];
            b += (u1 - u0) * (pretty ? 5 : 4);
            str += cols->url_off[u1] - cols->url_off[u0];
        }
        if (cols->tag_off) {
            const uint64_t t0 = cols->tag_off[0], t1 = cols->tag_off[n];
            b += (t1 - t0) * (pretty ? 96 : 64);
            str += cols->tag_name_off[t1] - cols->tag_name_off[t0];
        }
    }
    *bound = b + 6 * str;
    return PJ_OK;
}

void pj_decode_bounds(uint64_t len, pj_pet_columns *c) {
    if (!c) return;
    // a valid record needs at least {"name":"","photoUrls":[]} (26 bytes) + '\n'
    c->cap_pets = len / 27 + 1;
    c->cap_name_bytes = len;
    c->cap_cat_name_bytes = len;
    c->cap_urls = len / 3 + 1;      // each url needs "" and a separator
    c->cap_url_bytes = len;
    c->cap_tags = len / 3 + 1;      // each tag needs {} and a separator
    c->cap_tag_name_bytes = len;
}

}  // extern "C"

namespace {


constexpr uint64_t VLB_WORDS = PJ_DEC_NCNT;   // vector look-back words per line block

bool dec_cols_ok(const pj_pet_columns *o) {
    void *v[17];
    col_ptrs(const_cast<pj_pet_columns *>(o), v);
    for (void *x : v)
        if (!x) return false;
    return true;
}

// NDJSON (array = false) or one array document (array = true): the line
// stages are the same, only the index stage differs (newlines, or the
// array's frame: its elements' starts).
// The record index: the start of every NDJSON line, or of every element of
// one array document, built in ctx->index (X: its header words; 2 holds the
// record count).  Fills P's index fields (and zeroes the rest of P); the
// record count goes to *lines.  The array frame's verdict is checked here.
// With `cut` (array documents only) the frame is only scanned, for a
// document cut short: *cut gets the position of its last top-level comma
// (~0 when it has none), and no frame check is made.
pj_status index_stage(pj_ctx *ctx, const uint8_t *in, uint64_t len, bool array, DecParams &P, uint64_t *&X,
                      uint64_t *lines_out, uint64_t *cut = nullptr) {
    pj_status s;
    const uint64_t nblk64 = (len + 63) / 64;
    uint64_t ls_cap = len / 128 + 16;
    for (int attempt = 0; attempt < 2; attempt++) {
        // look-back words: one per block of the kernel that builds the index
        // (the newline index's, or the array frame's blocks)
        const uint64_t ga = array ? pj_arr_blocks(nblk64) : 0;
        const uint64_t gidx = std::max((nblk64 + pj_dec_index_block() - 1) / pj_dec_index_block(), ga);
        // layout (u64 units): header 16 | dummy 32 | array frame scalars 8 |
        //   state_idx gidx | (arrays: block summaries, entry states, per-thread
        //   summaries) | line_start ls_cap
        // header: 0-1 tickets, 2 line count, 3 blank lines, 4-11 totals,
        //         12 lines off the fast path, 13 deferred error-code queue
        //         length, 14 lines for k_dec_long, 15 scan ticket
        const uint64_t o_dummy = 16, o_arr = 48, o_sidx = 56;
        const uint64_t o_bsum = o_sidx + gidx, o_bpre = o_bsum + (ga * sizeof(FS) + 7) / 8;
        const uint64_t o_tsum = o_bpre + ga, ta = array ? pj_arr_threads(nblk64) : 0;
        const uint64_t o_ls = o_tsum + (ta * sizeof(FS) + 7) / 8;
        PJ_HIP(ctx->index.ensure((o_ls + ls_cap) * 8 + 64));
        X = static_cast<uint64_t *>(ctx->index.p);
        std::memset(&P, 0, sizeof P);
        P.in = in;
        P.len = len;
        P.nblk64 = nblk64;
        P.line_start = X + o_ls;
        P.ls_cap = ls_cap;
        P.n_lines = X + 2;
        P.totals = X + 4;
        P.state_idx = X + o_sidx;
        P.tickets = reinterpret_cast<unsigned long long *>(X);
        P.dummy = reinterpret_cast<uint32_t *>(X + o_dummy);
        P.gq_count = reinterpret_cast<unsigned long long *>(X + 12);
        P.empty_count = reinterpret_cast<unsigned long long *>(X + 3);
        P.array_doc = array ? 1 : 0;
        P.arr = X + o_arr;
        P.arr_bsum = reinterpret_cast<FS *>(X + o_bsum);
        P.arr_bpre = X + o_bpre;
        P.arr_tsum = reinterpret_cast<FS *>(X + o_tsum);
        // blocks in launch order with bounded look-back waits; a kernel
        // whose wait ran out (its ticket word set) is redone in ticket order
        P.order_by_id = 1;
        P.spin_limit = spin_limit();
        for (;;) {
            ctx->n_ev = 0;
            if ((s = mark(ctx))) return s;
            PJ_HIP(pj_launch_fill_u64(X, 16, 0, ctx->stream));
            PJ_HIP(pj_launch_fill_u64(X + o_sidx, gidx, 0, ctx->stream));
            if (array) {
                PJ_HIP(pj_launch_fill_u64(X + o_arr, 8, 0, ctx->stream));
                PJ_HIP(pj_launch_fill_u64(X + o_arr, 1, ~0ull, ctx->stream));      // first non-whitespace
                PJ_HIP(pj_launch_fill_u64(X + o_arr + 2, 1, ~0ull, ctx->stream));  // the close
            }
            if ((s = mark(ctx))) return s;
            if (array) PJ_HIP(pj_launch_arr_frame(P, ctx->stream));
            else if (nblk64) PJ_HIP(pj_launch_dec_index(P, ctx->stream));
            if ((s = mark(ctx))) return s;
            PJ_HIP(hipMemcpyAsync(ctx->pinned, X, 3 * sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
            if (array) PJ_HIP(hipMemcpyAsync(ctx->pinned + 16, X + o_arr, 8 * sizeof(uint64_t), hipMemcpyDeviceToHost,
                                             ctx->stream));
            PJ_HIP(hipStreamSynchronize(ctx->stream));
            if (array || !P.order_by_id || ctx->pinned[0] == 0) break;
            P.order_by_id = 0;
        }
        if (cut) {
            const uint64_t nsep = ctx->pinned[16 + 3];
            if (nsep + 2 > ls_cap) {       // the separators' starts did not all fit: grow and redo
                ls_cap = nsep + 2;
                continue;
            }
            *cut = ~0ull;
            if (nsep) {
                PJ_HIP(hipMemcpy(ctx->pinned, P.line_start + nsep, sizeof(uint64_t), hipMemcpyDeviceToHost));
                *cut = ctx->pinned[0] - 1;
            }
            return PJ_OK;
        }
        if (array && ctx->pinned[16 + 4] == 0) {
            (void)finish_timing(ctx);
            return fail(PJ_ERR_SYNTAX, "not a JSON array: '[', the top-level commas or the closing ']' are malformed");
        }
        const uint64_t lines = ctx->pinned[2];
        if (lines + 1 > ls_cap) {          // more lines than the first guess: grow and redo
            ls_cap = lines + 2;
            continue;
        }
        *lines_out = lines;
        return PJ_OK;
    }
    return fail(PJ_ERR_DEVICE, "line index did not converge");
}

pj_status decode_impl(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
                      uint8_t *err_code, uint64_t err_cap, pj_decode_result *res, bool array = false) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!out || !res) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (len && !in) return fail(PJ_ERR_INVALID_ARG, "null input");
    if (!dec_cols_ok(out)) return fail(PJ_ERR_INVALID_ARG, "decode needs every column pointer");
    if (err_cap && (!err_line || !err_code)) return fail(PJ_ERR_INVALID_ARG, "null error arrays");
    std::memset(res, 0, sizeof *res);
    ctx->n_ev = 0;
    DecParams P;
    uint64_t *X = nullptr, lines = 0;
    if ((s = index_stage(ctx, in, len, array, P, X, &lines))) return s;
    P.lines = lines;
    if (len >= PJ_DEC_MAX_BLOCK_SPAN && lines) {
        // the lines of one block must span less than 4 GiB (32-bit offsets
        // inside a block); only an input that long can break it
        PJ_HIP(pj_launch_fill_u64(X + 15, 1, 0, ctx->stream));
        PJ_HIP(pj_launch_dec_span_check(P, X + 15, ctx->stream));
        PJ_HIP(hipMemcpyAsync(ctx->pinned, X + 15, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->pinned[0]) {
            ctx->n_ev = 0;
            return fail(PJ_ERR_INVALID_ARG, "lines of 4 GiB or more in one block of " +
                                                std::to_string(pj_dec_parse_block()) + " lines (offsets inside a "
                                                "block are 32-bit)");
        }
    }
    P.o = *out;
    P.err_line = err_line;
    P.err_code = err_code;
    P.err_cap = err_cap;
    P.lines = lines;
    const uint64_t gp = (lines + pj_dec_parse_block() - 1) / pj_dec_parse_block();
    // the line tape (256 bytes per line), when it fits a modest bound;
    // with it the decode is split at the scan (the validating kernel
    // stores per-line offsets, the writers follow a block scan), without
    // it the single-pass kernel walks each line again to write it
    P.tape = nullptr;
    if (lines && decode_tape_enabled() && lines * 256 <= (16ull << 30) &&
        ctx->tape.ensure(lines * 256) == hipSuccess)
        P.tape = static_cast<uint64_t *>(ctx->tape.p);
    (void)hipGetLastError();
    const bool split = P.tape != nullptr;
    // scan buffer: vector look-back words (single pass) or block totals,
    // bases and scan look-back words (split), then the deferred
    // error-code queue, then (split) the wave-line list, the per-line
    // offsets (9 u32 per line), the count and list of blocks handed to
    // the bitmap pass
    const uint64_t nsb = (gp + pj_dec_bscan_block() - 1) / pj_dec_bscan_block();
    const uint64_t w_state = split ? 2 * gp * VLB_WORDS + nsb * VLB_WORDS : gp * VLB_WORDS;
    const uint64_t w_lpos = (9 * lines + 1) / 2;
    const uint64_t w_split = split ? lines + w_lpos + 2 + gp : 0;
    PJ_HIP(ctx->scan.ensure((w_state + lines + 8 + w_split) * 8));
    uint64_t *SB = static_cast<uint64_t *>(ctx->scan.p);
    P.state_parse = SB;
    P.bagg = SB;
    P.bbase = SB + gp * VLB_WORDS;
    P.bstate = SB + 2 * gp * VLB_WORDS;
    P.nblocks = gp;
    P.dq = SB + w_state;
    P.dq_count = reinterpret_cast<unsigned long long *>(X + 13);
    P.long_count = reinterpret_cast<unsigned long long *>(X + 14);
    P.bticket = reinterpret_cast<unsigned long long *>(X + 15);
    P.long_list = P.dq + lines + 8;
    P.lpos = reinterpret_cast<uint32_t *>(P.long_list + lines);
    P.bm_count = reinterpret_cast<unsigned long long *>(P.long_list + lines + w_lpos);
    P.bm_list = P.long_list + lines + w_lpos + 2;
    P.order_by_id = 1;
    for (;;) {
        if ((s = mark(ctx))) return s;
        if (split) {
            PJ_HIP(pj_launch_fill_u64(P.bstate, nsb * VLB_WORDS, 0, ctx->stream));
            PJ_HIP(pj_launch_fill_u64(reinterpret_cast<uint64_t *>(P.bm_count), 2, 0, ctx->stream));
        }
        else PJ_HIP(pj_launch_fill_u64(P.state_parse, gp * VLB_WORDS, 0, ctx->stream));
        PJ_HIP(pj_launch_fill_u64(X + 1, 1, 0, ctx->stream));      // the parse ticket / give-up word
        PJ_HIP(pj_launch_fill_u64(X + 3, 13, 0, ctx->stream));     // totals and counters
        if ((s = mark(ctx))) return s;
        if (lines) {
            PJ_HIP(pj_launch_dec_parse(P, ctx->stream));
            if (split) {
                if ((s = mark(ctx))) return s;
                PJ_HIP(pj_launch_dec_bscan(P, ctx->stream));
                if ((s = mark(ctx))) return s;
                PJ_HIP(pj_launch_dec_write(P, ctx->stream));
                if ((s = mark(ctx))) return s;
                PJ_HIP(pj_launch_dec_long(P, ctx->stream));
            }
            if ((s = mark(ctx))) return s;
            PJ_HIP(pj_launch_dec_errcode(P, ctx->stream));
        } else {
            // no lines: the offset arrays still start with 0
            uint64_t *heads[6] = {out->name_off, out->cat_name_off, out->photo_off, out->tag_off, out->url_off,
                                  out->tag_name_off};
            for (uint64_t *h : heads) PJ_HIP(pj_launch_fill_u64(h, 1, 0, ctx->stream));
        }
        if ((s = mark(ctx))) return s;
        PJ_HIP(hipMemcpyAsync(ctx->pinned, X, 13 * sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        if (!P.order_by_id || ctx->pinned[1] == 0) break;
        P.order_by_id = 0;
        ctx->n_ev = 0;
    }
    if ((s = finish_timing(ctx))) return s;
    const uint64_t *T = ctx->pinned + 4;
    res->n_general = lines ? ctx->pinned[12] : 0;
    res->n_lines = lines;
    if (array && lines && ctx->pinned[3]) {
        // a blank element: "[ ]" holds none, any other is a broken frame
        if (lines > 1) return fail(PJ_ERR_SYNTAX, "an element of the array is empty");
        std::memset(res, 0, sizeof *res);
        out->n_pets = 0;
        return PJ_OK;
    }
    if (lines) {
        res->n_pets = T[C_PETS];
        res->name_bytes = T[C_NAMEB];
        res->cat_name_bytes = T[C_CATB];
        res->n_urls = T[C_URLS];
        res->url_bytes = T[C_URLB];
        res->n_tags = T[C_TAGS];
        res->tag_name_bytes = T[C_TAGB];
        res->n_errors = T[C_ERRS];
    }
    out->n_pets = std::min(res->n_pets, out->cap_pets);
    if (res->n_errors > err_cap) return fail(PJ_ERR_CAPACITY, "error list capacity too small");
    if (res->n_pets > out->cap_pets || res->name_bytes > out->cap_name_bytes ||
        res->cat_name_bytes > out->cap_cat_name_bytes || res->n_urls > out->cap_urls ||
        res->url_bytes > out->cap_url_bytes || res->n_tags > out->cap_tags ||
        res->tag_name_bytes > out->cap_tag_name_bytes)
        return fail(PJ_ERR_CAPACITY, "column capacity too small (sizes needed are in the result)");
    return PJ_OK;
}

}  // namespace

extern "C" pj_status pj_decode_device(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out,
                                      uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
                                      pj_decode_result *res) {
    return decode_impl(ctx, in, len, out, err_line, err_code, err_cap, res);
}

extern "C" pj_status pj_decode_array_device(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out,
                                            uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
                                            pj_decode_result *res) {
    return decode_impl(ctx, in, len, out, err_line, err_code, err_cap, res, true);
}

namespace {
pj_status decode_host_impl(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
                           uint8_t *err_code, uint64_t err_cap, pj_decode_result *res, bool array);
}

extern "C" void *pj_host_alloc(uint64_t n) {
    void *p = nullptr;
    if (hipHostMalloc(&p, n ? n : 1, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

extern "C" void pj_host_free(void *p) {
    if (p) (void)hipHostFree(p);
}

extern "C" pj_status pj_decode_host(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out,
                                    uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
                                    pj_decode_result *res) {
    return decode_host_impl(ctx, in, len, out, err_line, err_code, err_cap, res, false);
}

extern "C" pj_status pj_decode_array_host(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out,
                                          uint64_t *err_line, uint8_t *err_code, uint64_t err_cap,
                                          pj_decode_result *res) {
    return decode_host_impl(ctx, in, len, out, err_line, err_code, err_cap, res, true);
}

namespace {
// Streamed host decode: an NDJSON input of more than stream_above() bytes
// is decoded in segments of about segment_bytes(), cut after a newline, in
// a three-stage pipeline: while segment k decodes on the context stream, a
// host thread copies segment k + 1 in (copy engine xin) and another copies
// segment k - 1's columns out (copy engine xout) to the caller's arrays at
// the running offsets, its offset arrays and error line numbers shifted on
// the device first.  Both copy directions run at once (PCIe is full
// duplex), each through its own pinned bounce buffers.  Device memory is
// bounded by two segments and their outputs, not by the input.
uint64_t segment_bytes() {
    if (const char *e = std::getenv("PETJSON_DECODE_SEGMENT")) {
        const unsigned long long v = std::strtoull(e, nullptr, 10);
        if (v) return v;
    }
    return 256ull << 20;
}
uint64_t stream_above() {
    if (std::getenv("PETJSON_DECODE_SEGMENT")) return segment_bytes();
    return 2 * segment_bytes();
}

// Device layout of one segment's outputs: the 17 columns (sized for n
// input bytes) and the error list (ce entries).
struct SegOut {
    uint64_t off[20];
    uint64_t cp, cu, ct;
    pj_pet_columns dc;
};
SegOut seg_layout(uint64_t n, uint64_t ce) {
    SegOut L;
    std::memset(&L.dc, 0, sizeof L.dc);
    pj_decode_bounds(n, &L.dc);
    L.cp = L.dc.cap_pets;
    L.cu = L.dc.cap_urls;
    L.ct = L.dc.cap_tags;
    const uint64_t cp = L.cp, cu = L.cu, ct = L.ct;
    const uint64_t sz[19] = {cp * 8, cp, cp, (cp + 1) * 8, L.dc.cap_name_bytes, cp * 8, cp, (cp + 1) * 8,
                             L.dc.cap_cat_name_bytes, (cp + 1) * 8, (cu + 1) * 8, L.dc.cap_url_bytes, (cp + 1) * 8,
                             ct * 8, ct, (ct + 1) * 8, L.dc.cap_tag_name_bytes, ce * 8, ce};
    L.off[0] = 0;
    for (int j = 0; j < 19; j++) L.off[j + 1] = L.off[j] + align256(sz[j] + 8);
    return L;
}

// Array documents stream too: segment k after the first is the bytes after
// a top-level comma, behind a '[' written in front of them on the device.
// Where the segment can end is only known once it is on the device: the
// frame scan of the cut document gives its last top-level comma, which
// becomes a ']' so that the segment is a whole document of the elements up
// to it (a segment with no such comma is loaded again twice as long); the
// next segment starts after that comma.  Its elements are numbered on from
// the earlier segments', as lines are.  (A frame error is reported as by
// the one-shot decode when it shows inside one segment's document.)
pj_status array_segment(pj_ctx *ctx, const uint8_t *in, uint64_t len, uint64_t a, uint64_t seg, int k, DevBuf &buf,
                        uint64_t *n, uint64_t *next) {
    const uint64_t pre = k == 0 && a == 0 ? 0 : 1;
    for (uint64_t Z = std::min(seg, len - a);; Z = std::min(2 * Z, len - a)) {
        PJ_HIP(buf.ensure(pre + Z + 16));
        uint8_t *D = static_cast<uint8_t *>(buf.p);
        pj_status s;
        if ((s = h2d(ctx, D + pre, in + a, Z))) return s;
        if (pre) PJ_HIP(pj_launch_put_bytes(D, '[', 1, ctx->stream));
        if (a + Z == len) {           // the document's own end
            *n = pre + Z;
            *next = len;
            return PJ_OK;
        }
        DecParams P;
        uint64_t *X, lines, cut = ~0ull;
        if ((s = index_stage(ctx, D, pre + Z, true, P, X, &lines, &cut))) return s;
        if (cut != ~0ull && cut >= pre) {
            PJ_HIP(pj_launch_put_bytes(D + cut, ']', 1, ctx->stream));
            *n = cut + 1;
            *next = a + (cut - pre) + 1;
            return PJ_OK;
        }
    }
}

pj_status decode_host_stream(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
                             uint8_t *err_code, uint64_t err_cap, pj_decode_result *res, bool array) {
    const uint64_t seg = segment_bytes();
    // segments end after a newline (or at the end); a line longer than a
    // segment makes its segment longer
    auto seg_end = [&](uint64_t a) -> uint64_t {
        if (len - a <= seg) return len;
        const void *p = memrchr(in + a, '\n', seg);
        if (p) return (uint64_t)(static_cast<const uint8_t *>(p) - in) + 1;
        const void *q = std::memchr(in + a + seg, '\n', len - a - seg);
        return q ? (uint64_t)(static_cast<const uint8_t *>(q) - in) + 1 : len;
    };
    std::memset(res, 0, sizeof *res);
    if (!ctx->seg_ready) PJ_HIP(hipEventCreateWithFlags(&ctx->seg_ready, hipEventDisableTiming));
    uint64_t base[PJ_DEC_NCNT] = {0, 0, 0, 0, 0, 0, 0, 0};   // rows, bytes and items written before the segment
    uint64_t lines = 0;
    bool over = false;                 // the caller's capacities ran out: only counting from there
    pj_status s = PJ_OK;
    DevBuf *stage[2] = {&ctx->stage_out, &ctx->stage_out2};
    // buffers for a full segment, sized once (a longer segment, cut after a
    // long line, grows them)
    const uint64_t ce0 = seg / 16 + 16;   // the error list: a first guess, redone once with the count
    PJ_HIP(ctx->seg_in[0].ensure(std::min(seg, len) + 16));
    PJ_HIP(ctx->seg_in[1].ensure(std::min(seg, len) + 16));
    {
        const SegOut L = seg_layout(std::min(seg, len), ce0);
        PJ_HIP(stage[0]->ensure(L.off[19]));
        PJ_HIP(stage[1]->ensure(L.off[19]));
    }
    // a host thread's result
    struct Job {
        std::thread th;
        pj_status st = PJ_OK;
        std::string err;
        pj_status join() {
            if (th.joinable()) th.join();
            const pj_status r = st;
            st = PJ_OK;
            return r;
        }
    };
    Job cin, cout;
    auto finish = [&](pj_status r) -> pj_status {
        const pj_status a1 = cin.join(), a2 = cout.join();
        if (r) return r;
        if (a1) return fail(a1, cin.err);
        if (a2) return fail(a2, cout.err);
        return PJ_OK;
    };
    uint64_t a = 0, b = 0;
    uint64_t an = 0, anext = 0;      // arrays: this segment's bytes on the device, the next one's start
    // the first segment in
    if (array) {
        if ((s = array_segment(ctx, in, len, 0, seg, 0, ctx->seg_in[0], &an, &anext))) return s;
    } else {
        b = seg_end(0);
        if ((s = h2d(ctx, static_cast<uint8_t *>(ctx->seg_in[0].p), in, b - a, false))) return s;
    }
    for (int k = 0; a < len; k ^= 1) {
        const uint64_t n = array ? an : b - a;
        const uint64_t a2 = array ? anext : b, b2 = array ? 0 : (b < len ? seg_end(b) : b);
        // the next segment in, while this one decodes (NDJSON: its end is
        // known on the host)
        if (!array && a2 < len) {
            if (ctx->seg_in[k ^ 1].ensure(b2 - a2 + 16) != hipSuccess) return finish(fail(PJ_ERR_DEVICE, "segment buffer"));
            cin.th = std::thread([&, k, a2, b2] {
                pj_status r = bind(ctx);               // (HIP's current device is per thread)
                if (!r) r = h2d(ctx, static_cast<uint8_t *>(ctx->seg_in[k ^ 1].p), in + a2, b2 - a2, false);
                if (r) cin.err = pj_last_error();
                cin.st = r;
            });
        }
        // this segment: columns sized for it in this slot's staging (segment
        // k - 2's copy-out, which used it, was joined one segment ago)
        uint64_t ce = ce0;
        SegOut L;
        pj_decode_result r;
      again:
        L = seg_layout(n, ce);
        if (stage[k]->ensure(L.off[19]) != hipSuccess) return finish(fail(PJ_ERR_DEVICE, "segment columns: out of device memory"));
        uint8_t *D = static_cast<uint8_t *>(stage[k]->p);
        {
            void *dp[17];
            for (int j = 0; j < 17; j++) dp[j] = D + L.off[j];
            set_col_ptrs(&L.dc, dp);
        }
        uint64_t *del = reinterpret_cast<uint64_t *>(D + L.off[17]);
        uint8_t *dec = D + L.off[18];
        s = decode_impl(ctx, static_cast<uint8_t *>(ctx->seg_in[k].p), n, &L.dc, del, dec, ce, &r, array);
        if (s == PJ_ERR_CAPACITY && r.n_errors > ce) {
            ce = r.n_errors;
            goto again;
        }
        if (s) return finish(s);
        const uint64_t T[PJ_DEC_NCNT] = {r.n_pets, r.name_bytes, r.cat_name_bytes, r.n_urls,
                                         r.url_bytes, r.n_tags, r.tag_name_bytes, r.n_errors};
        over = over || base[C_PETS] + T[C_PETS] > out->cap_pets || base[C_NAMEB] + T[C_NAMEB] > out->cap_name_bytes ||
               base[C_CATB] + T[C_CATB] > out->cap_cat_name_bytes || base[C_URLS] + T[C_URLS] > out->cap_urls ||
               base[C_URLB] + T[C_URLB] > out->cap_url_bytes || base[C_TAGS] + T[C_TAGS] > out->cap_tags ||
               base[C_TAGB] + T[C_TAGB] > out->cap_tag_name_bytes || base[C_ERRS] + T[C_ERRS] > err_cap;
        // segment k - 1's copy-out is done before this one's starts (one
        // copy engine out); its staging slot is then free for segment k + 1
        if (const pj_status c1 = cout.join()) return finish(fail(c1, cout.err));
        if (!over) {
            // offsets and error lines shifted past the earlier segments, then out
            const uint64_t np = T[C_PETS];
            hipError_t x;
            if ((x = pj_launch_add_u64(L.dc.name_off, np + 1, base[C_NAMEB], ctx->stream)) ||
                (x = pj_launch_add_u64(L.dc.cat_name_off, np + 1, base[C_CATB], ctx->stream)) ||
                (x = pj_launch_add_u64(L.dc.photo_off, np + 1, base[C_URLS], ctx->stream)) ||
                (x = pj_launch_add_u64(L.dc.tag_off, np + 1, base[C_TAGS], ctx->stream)) ||
                (x = pj_launch_add_u64(L.dc.url_off, T[C_URLS] + 1, base[C_URLB], ctx->stream)) ||
                (x = pj_launch_add_u64(L.dc.tag_name_off, T[C_TAGS] + 1, base[C_TAGB], ctx->stream)) ||
                (x = pj_launch_add_u64(del, T[C_ERRS], lines, ctx->stream)) ||
                (x = hipEventRecord(ctx->seg_ready, ctx->stream)))
                return finish(fail(PJ_ERR_DEVICE, std::string("segment offsets: ") + hipGetErrorString(x)));
            // host destination of each column: its element at the running base
            void *hp[17];
            col_ptrs(out, hp);
            const uint64_t nu = r.n_urls, nt = r.n_tags;
            const uint64_t bp = base[C_PETS], bu = base[C_URLS], bt = base[C_TAGS];
            struct Piece { uint8_t *dst; const uint8_t *src; uint64_t n; };
            std::vector<Piece> pieces;
            const uint64_t dst_off[17] = {bp * 8, bp, bp, bp * 8, base[C_NAMEB], bp * 8, bp, bp * 8, base[C_CATB],
                                          bp * 8, bu * 8, base[C_URLB], bp * 8, bt * 8, bt, bt * 8, base[C_TAGB]};
            const uint64_t used[17] = {np * 8, np, np, (np + 1) * 8, r.name_bytes, np * 8, np, (np + 1) * 8,
                                       r.cat_name_bytes, (np + 1) * 8, (nu + 1) * 8, r.url_bytes, (np + 1) * 8,
                                       nt * 8, nt, (nt + 1) * 8, r.tag_name_bytes};
            for (int j = 0; j < 17; j++)
                if (used[j]) pieces.push_back({static_cast<uint8_t *>(hp[j]) + dst_off[j], D + L.off[j], used[j]});
            if (r.n_errors) {
                pieces.push_back({reinterpret_cast<uint8_t *>(err_line + base[C_ERRS]), D + L.off[17], r.n_errors * 8});
                pieces.push_back({err_code + base[C_ERRS], D + L.off[18], r.n_errors});
            }
            // every piece waits for the event as recorded now, never for the
            // context stream, where the next segment is being queued (the next
            // record of the event comes after this thread is joined)
            hipEvent_t ready = ctx->seg_ready;
            cout.th = std::thread([&, pieces, ready] {
                pj_status q = bind(ctx);
                for (size_t j = 0; !q && j < pieces.size(); j++)
                    q = d2h(ctx, pieces[j].dst, pieces[j].src, pieces[j].n, ready, false);
                if (!q) q = d2h_wait(ctx);
                if (q) cout.err = pj_last_error();
                cout.st = q;
            });
        }
        base[C_PETS] += r.n_pets; base[C_NAMEB] += r.name_bytes; base[C_CATB] += r.cat_name_bytes;
        base[C_URLS] += r.n_urls; base[C_URLB] += r.url_bytes; base[C_TAGS] += r.n_tags;
        base[C_TAGB] += r.tag_name_bytes; base[C_ERRS] += r.n_errors;
        lines += r.n_lines;
        res->n_general += r.n_general;
        // the next segment is on the device before it decodes
        if (const pj_status c2 = cin.join()) return finish(fail(c2, cin.err));
        if (array && a2 < len) {
            if ((s = array_segment(ctx, in, len, a2, seg, k ^ 1, ctx->seg_in[k ^ 1], &an, &anext))) return finish(s);
        }
        a = a2;
        b = b2;
    }
    if ((s = finish(PJ_OK))) return s;
    res->n_lines = lines;
    res->n_pets = base[C_PETS]; res->name_bytes = base[C_NAMEB]; res->cat_name_bytes = base[C_CATB];
    res->n_urls = base[C_URLS]; res->url_bytes = base[C_URLB]; res->n_tags = base[C_TAGS];
    res->tag_name_bytes = base[C_TAGB]; res->n_errors = base[C_ERRS];
    if (over) {
        out->n_pets = 0;
        return fail(PJ_ERR_CAPACITY, "capacity too small (sizes needed are in the result)");
    }
    out->n_pets = res->n_pets;
    return PJ_OK;
}

pj_status decode_host_impl(pj_ctx *ctx, const uint8_t *in, uint64_t len, pj_pet_columns *out, uint64_t *err_line,
                           uint8_t *err_code, uint64_t err_cap, pj_decode_result *res, bool array) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!out || !res) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (len && !in) return fail(PJ_ERR_INVALID_ARG, "null input");
    if (!dec_cols_ok(out)) return fail(PJ_ERR_INVALID_ARG, "decode needs every column pointer");
    if (err_cap && (!err_line || !err_code)) return fail(PJ_ERR_INVALID_ARG, "null error arrays");
    if (len > stream_above()) return decode_host_stream(ctx, in, len, out, err_line, err_code, err_cap, res, array);
    // device staging: input, then every output column sized by the capacities
    const uint64_t cp = out->cap_pets, cu = out->cap_urls, ct = out->cap_tags;
    const uint64_t sz[19] = {cp * 8, cp, cp, (cp + 1) * 8, out->cap_name_bytes, cp * 8, cp, (cp + 1) * 8,
                             out->cap_cat_name_bytes, (cp + 1) * 8, (cu + 1) * 8, out->cap_url_bytes, (cp + 1) * 8,
                             ct * 8, ct, (ct + 1) * 8, out->cap_tag_name_bytes, err_cap * 8, err_cap};
    uint64_t off[20];
    off[0] = align256(len + 16);
    for (int k = 0; k < 19; k++) off[k + 1] = off[k] + align256(sz[k] + 8);
    PJ_HIP(ctx->stage_out.ensure(off[19]));
    uint8_t *D = static_cast<uint8_t *>(ctx->stage_out.p);
    if (len && (s = h2d(ctx, D, in, len))) return s;
    void *dp[17];
    for (int k = 0; k < 17; k++) dp[k] = D + off[k];
    pj_pet_columns dc = *out;
    set_col_ptrs(&dc, dp);
    uint64_t *del = reinterpret_cast<uint64_t *>(D + off[17]);
    uint8_t *dec = D + off[18];
    s = decode_impl(ctx, D, len, &dc, err_cap ? del : nullptr, err_cap ? dec : nullptr, err_cap, res, array);
    if (s != PJ_OK && s != PJ_ERR_CAPACITY) return s;
    const uint64_t np = std::min(res->n_pets, cp), nu = std::min(res->n_urls, cu), nt = std::min(res->n_tags, ct);
    const uint64_t used[17] = {np * 8, np, np, (np + 1) * 8, std::min(res->name_bytes, out->cap_name_bytes), np * 8,
                               np, (np + 1) * 8, std::min(res->cat_name_bytes, out->cap_cat_name_bytes),
                               (np + 1) * 8, (nu + 1) * 8, std::min(res->url_bytes, out->cap_url_bytes),
                               (np + 1) * 8, nt * 8, nt, (nt + 1) * 8,
                               std::min(res->tag_name_bytes, out->cap_tag_name_bytes)};
    void *hp[17];
    col_ptrs(out, hp);
    pj_status t = PJ_OK;
    for (int k = 0; k < 17; k++)
        if (used[k] && (t = d2h(ctx, hp[k], dp[k], used[k], nullptr, false))) return t;
    const uint64_t ne = std::min(res->n_errors, err_cap);
    if (ne && ((t = d2h(ctx, err_line, del, ne * 8, nullptr, false)) || (t = d2h(ctx, err_code, dec, ne, nullptr, false))))
        return t;
    if ((t = d2h_wait(ctx))) return t;
    out->n_pets = np;
    return s;
}
}  // namespace

// ------------------------------------------------------ Order and User models
namespace {
bool model_ok(int m) { return m == PJ_MODEL_ORDER || m == PJ_MODEL_USER; }
int model_props(int m) { return m == PJ_MODEL_ORDER ? 6 : 8; }
bool model_str(int m, int k) { return m == PJ_MODEL_ORDER ? k == 3 : (k >= 1 && k <= 6); }

pj_status check_model_cols(int model, const pj_model_columns *c, bool decode) {
    for (int k = 0; k < model_props(model); k++) {
        if (!c->col[k]) return fail(PJ_ERR_INVALID_ARG, "model column " + std::to_string(k) + " missing");
        if (model_str(model, k) && !c->bytes[k])
            return fail(PJ_ERR_INVALID_ARG, "model string column " + std::to_string(k) + " has no bytes");
    }
    if (decode && !c->present) return fail(PJ_ERR_INVALID_ARG, "decode needs the present column");
    return PJ_OK;
}
}  // namespace

extern "C" pj_status pj_encode_model_device(pj_ctx *ctx, int model, const pj_model_columns *cols, int format,
                                            uint8_t *out, uint64_t out_cap, uint64_t *out_len) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!model_ok(model)) return fail(PJ_ERR_INVALID_ARG, "unknown model");
    if (!format_ok(format)) return fail(PJ_ERR_INVALID_ARG, "bad format");
    if (out_cap > 0 && !out) return fail(PJ_ERR_INVALID_ARG, "null output with capacity");
    const uint64_t n = cols->n;
    if (n && (s = check_model_cols(model, cols, false))) return s;
    ctx->n_ev = 0;
    if (n == 0) {
        const uint64_t len = format == PJ_FORMAT_ARRAY ? 2 : format == PJ_FORMAT_PRETTY ? 3 : 0;
        *out_len = len;
        if (len && len <= out_cap) {
            const uint32_t w = format == PJ_FORMAT_ARRAY ? '[' | (']' << 8) : '[' | (' ' << 8) | (']' << 16);
            PJ_HIP(pj_launch_put_bytes(out, w, (int)len, ctx->stream));
        }
        PJ_HIP(hipStreamSynchronize(ctx->stream));
        return len > out_cap ? fail(PJ_ERR_CAPACITY, "output capacity too small") : PJ_OK;
    }
    const uint64_t bt = (uint64_t)pj_encode_model_records(), nblk = (n + bt - 1) / bt;
    PJ_HIP(ctx->scan.ensure((nblk + 2) * sizeof(uint64_t)));
    uint64_t *sc = static_cast<uint64_t *>(ctx->scan.p);
    ModelEncParams P;
    std::memset(&P, 0, sizeof P);
    P.c = *cols;
    P.n = n;
    P.model = model;
    P.format = format;
    P.incl = (uint32_t)ctx->opt.inclusion;
    P.hexa = ctx->opt.hex_upper ? 'A' : 'a';
    P.out = out;
    P.cap = out_cap;
    P.ticket = reinterpret_cast<unsigned long long *>(sc);
    P.total = sc + 1;
    P.state = sc + 2;
    if ((s = mark(ctx))) return s;
    PJ_HIP(pj_launch_fill_u64(sc, nblk + 2, 0, ctx->stream));
    if ((s = mark(ctx))) return s;
    PJ_HIP(pj_launch_encode_model(P, ctx->stream));
    if ((s = mark(ctx))) return s;
    PJ_HIP(hipMemcpyAsync(ctx->pinned, sc + 1, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
    PJ_HIP(hipStreamSynchronize(ctx->stream));
    if ((s = finish_timing(ctx))) return s;
    *out_len = ctx->pinned[0];
    if (*out_len > out_cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    return PJ_OK;
}

extern "C" pj_status pj_decode_model_device(pj_ctx *ctx, int model, const uint8_t *in, uint64_t len, int array,
                                            pj_model_columns *out, uint64_t *err_line, uint8_t *err_code,
                                            uint64_t err_cap, pj_decode_result *res) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!out || !res) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!model_ok(model)) return fail(PJ_ERR_INVALID_ARG, "unknown model");
    if (len && !in) return fail(PJ_ERR_INVALID_ARG, "null input");
    if ((s = check_model_cols(model, out, true))) return s;
    if (err_cap && (!err_line || !err_code)) return fail(PJ_ERR_INVALID_ARG, "null error arrays");
    std::memset(res, 0, sizeof *res);
    ctx->n_ev = 0;
    DecParams P;
    uint64_t *X = nullptr, lines = 0;
    if ((s = index_stage(ctx, in, len, array != 0, P, X, &lines))) return s;
    const uint64_t nb = (lines + pj_decode_model_block() - 1) / pj_decode_model_block();
    const uint64_t nchunks = (nb + 1023) / 1024;     // the scan's chunks of 1024 blocks
    PJ_HIP(ctx->scan.ensure((2 * nb * MD_MAXK + nchunks * MD_MAXK + MD_MAXK + 1) * sizeof(uint64_t)));
    uint64_t *SB = static_cast<uint64_t *>(ctx->scan.p);
    ModelDecParams M;
    std::memset(&M, 0, sizeof M);
    M.in = in;
    M.len = len;
    M.line_start = P.line_start;
    M.lines = lines;
    M.o = *out;
    M.err_line = err_line;
    M.err_code = err_code;
    M.err_cap = err_cap;
    M.totals = SB;
    M.bagg = SB + MD_MAXK + 1;
    M.bbase = M.bagg + nb * MD_MAXK;
    M.csum = M.bbase + nb * MD_MAXK;
    M.nblocks = nb;
    // the counting pass's record tape (one word per property and one for the
    // record), while it stays under 16 GiB
    const uint64_t tw = lines * (1 + (uint64_t)model_props(model));
    if (decode_tape_enabled() && lines && tw * 8 <= (16ull << 30)) {
        PJ_HIP(ctx->tape.ensure(tw * 8));
        M.tape = static_cast<uint64_t *>(ctx->tape.p);
    }
    if ((s = mark(ctx))) return s;
    PJ_HIP(pj_launch_fill_u64(SB, MD_MAXK + 1, 0, ctx->stream));
    for (int k = 0; k < model_props(model); k++)    // string offsets start at 0
        if (model_str(model, k)) PJ_HIP(pj_launch_fill_u64(static_cast<uint64_t *>(out->col[k]), 1, 0, ctx->stream));
    if ((s = mark(ctx))) return s;
    PJ_HIP(pj_launch_decode_model(M, model, ctx->stream));
    if ((s = mark(ctx))) return s;
    PJ_HIP(hipMemcpyAsync(ctx->pinned, SB, (MD_MAXK + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
    PJ_HIP(hipStreamSynchronize(ctx->stream));
    if ((s = finish_timing(ctx))) return s;
    const uint64_t *T = ctx->pinned;
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) out->n_bytes[k] = 0;
    if (array && lines && T[MD_MAXK]) {
        // a blank element: "[ ]" holds none, any other is a broken frame
        if (lines > 1) return fail(PJ_ERR_SYNTAX, "an element of the array is empty");
        out->n = 0;
        return PJ_OK;
    }
    res->n_lines = lines;
    res->n_pets = T[0];
    res->n_errors = T[1];
    out->n = std::min(T[0], out->cap_n);
    bool over = T[0] > out->cap_n;
    for (int k = 0; k < model_props(model); k++)
        if (model_str(model, k)) {
            out->n_bytes[k] = T[2 + k];
            over = over || T[2 + k] > out->cap_bytes[k];
        }
    if (res->n_errors > err_cap) return fail(PJ_ERR_CAPACITY, "error list capacity too small");
    if (over) return fail(PJ_ERR_CAPACITY, "column capacity too small (sizes needed are in the result)");
    return PJ_OK;
}

extern "C" void pj_decode_model_bounds(int model, uint64_t len, pj_model_columns *c) {
    if (!c) return;
    // a record needs at least "{}" and a separator
    c->cap_n = len / 3 + 1;
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++)
        c->cap_bytes[k] = model_ok(model) && k < model_props(model) && model_str(model, k) ? len : 0;
}

// ------------------------------------------------ Order and User, host memory
namespace {
// Bytes of column k of n records (string properties: the n + 1 offsets),
// and of its string bytes.
uint64_t model_col_bytes(int model, int k, uint64_t n) {
    if (model_str(model, k)) return (n + 1) * 8;
    const bool wide = k == 0 || (model == PJ_MODEL_ORDER && k == 1);       // int64 ids
    const bool i32 = (model == PJ_MODEL_ORDER && k == 2) || (model == PJ_MODEL_USER && k == 7);
    return n * (wide ? 8 : i32 ? 4 : 1);
}
}  // namespace

extern "C" pj_status pj_encode_model_host(pj_ctx *ctx, int model, const pj_model_columns *cols, int format,
                                          uint8_t *out, uint64_t out_cap, uint64_t *out_len) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!cols || !out_len) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!model_ok(model)) return fail(PJ_ERR_INVALID_ARG, "unknown model");
    const uint64_t n = cols->n;
    if (n && (s = check_model_cols(model, cols, false))) return s;
    // staging layout: present, then each column and its bytes
    pj_model_columns dc = *cols;
    uint64_t off = 0, o_present = 0, o_col[PJ_MODEL_MAX_PROPS] = {}, o_bytes[PJ_MODEL_MAX_PROPS] = {},
             nbytes[PJ_MODEL_MAX_PROPS] = {};
    if (cols->present) { o_present = off; off += align256(n + 4); }
    for (int k = 0; n && k < model_props(model); k++) {
        o_col[k] = off;
        off += align256(model_col_bytes(model, k, n) + 4);
        if (model_str(model, k)) {
            nbytes[k] = static_cast<const uint64_t *>(cols->col[k])[n];
            o_bytes[k] = off;
            off += align256(nbytes[k] + 8);
        }
    }
    PJ_HIP(ctx->stage_in.ensure(off + 256));
    uint8_t *base = static_cast<uint8_t *>(ctx->stage_in.p);
    if (cols->present) {
        dc.present = base + o_present;
        if ((s = h2d(ctx, dc.present, cols->present, n, true, false))) return s;
    }
    for (int k = 0; n && k < model_props(model); k++) {
        dc.col[k] = base + o_col[k];
        if ((s = h2d(ctx, dc.col[k], cols->col[k], model_col_bytes(model, k, n), true, false))) return s;
        if (model_str(model, k)) {
            dc.bytes[k] = base + o_bytes[k];
            if ((s = h2d(ctx, dc.bytes[k], cols->bytes[k], nbytes[k], true, false))) return s;
        }
    }
    if ((s = h2d_wait(ctx))) return s;
    uint64_t need = 0;
    s = pj_encode_model_device(ctx, model, &dc, format, nullptr, 0, &need);
    if (s != PJ_OK && s != PJ_ERR_CAPACITY) return s;
    *out_len = need;
    if (need > out_cap) return fail(PJ_ERR_CAPACITY, "output capacity too small");
    if (need == 0) return PJ_OK;
    if (!out) return fail(PJ_ERR_INVALID_ARG, "null output");
    PJ_HIP(ctx->stage_out.ensure(need + 4));
    uint64_t got = 0;
    if ((s = pj_encode_model_device(ctx, model, &dc, format, static_cast<uint8_t *>(ctx->stage_out.p), need, &got)))
        return s;
    if ((s = d2h(ctx, out, ctx->stage_out.p, got))) return s;
    *out_len = got;
    return PJ_OK;
}

extern "C" pj_status pj_decode_model_host(pj_ctx *ctx, int model, const uint8_t *in, uint64_t len, int array,
                                          pj_model_columns *out, uint64_t *err_line, uint8_t *err_code,
                                          uint64_t err_cap, pj_decode_result *res) {
    pj_status s = bind(ctx);
    if (s) return s;
    if (!out || !res) return fail(PJ_ERR_INVALID_ARG, "null argument");
    if (!model_ok(model)) return fail(PJ_ERR_INVALID_ARG, "unknown model");
    if (len && !in) return fail(PJ_ERR_INVALID_ARG, "null input");
    if ((s = check_model_cols(model, out, true))) return s;
    if (err_cap && (!err_line || !err_code)) return fail(PJ_ERR_INVALID_ARG, "null error arrays");
    // device outputs sized by the caller's capacities, then the errors
    const uint64_t cap = out->cap_n;
    pj_model_columns dc = *out;
    uint64_t off = 0, o_col[PJ_MODEL_MAX_PROPS] = {}, o_bytes[PJ_MODEL_MAX_PROPS] = {};
    const uint64_t o_present = off;
    off += align256(cap + 4);
    for (int k = 0; k < model_props(model); k++) {
        o_col[k] = off;
        off += align256(model_col_bytes(model, k, cap) + 8);
        if (model_str(model, k)) {
            o_bytes[k] = off;
            off += align256(out->cap_bytes[k] + 8);
        }
    }
    const uint64_t o_el = off, o_ec = o_el + align256(err_cap * 8 + 8);
    off = o_ec + align256(err_cap + 8);
    PJ_HIP(ctx->stage_out.ensure(off + 256));
    PJ_HIP(ctx->stage_in.ensure(len + 64));
    uint8_t *ob = static_cast<uint8_t *>(ctx->stage_out.p), *D = static_cast<uint8_t *>(ctx->stage_in.p);
    dc.present = ob + o_present;
    for (int k = 0; k < model_props(model); k++) {
        dc.col[k] = ob + o_col[k];
        if (model_str(model, k)) dc.bytes[k] = ob + o_bytes[k];
    }
    if (len && (s = h2d(ctx, D, in, len))) return s;
    uint64_t *del = reinterpret_cast<uint64_t *>(ob + o_el);
    uint8_t *dec = ob + o_ec;
    s = pj_decode_model_device(ctx, model, D, len, array, &dc, err_cap ? del : nullptr, err_cap ? dec : nullptr,
                               err_cap, res);
    if (s != PJ_OK && s != PJ_ERR_CAPACITY) return s;
    const pj_status ds = s;
    // what was written: the rows that fit, their string bytes, the errors listed
    const uint64_t rows = dc.n;
    out->n = rows;
    for (int k = 0; k < PJ_MODEL_MAX_PROPS; k++) out->n_bytes[k] = dc.n_bytes[k];
    pj_status t;
    if ((t = d2h(ctx, out->present, dc.present, rows, nullptr, false))) return t;
    for (int k = 0; k < model_props(model); k++) {
        if (model_str(model, k)) {
            if ((t = d2h(ctx, out->col[k], dc.col[k], (rows + 1) * 8, nullptr, false))) return t;
            const uint64_t nb = std::min(dc.n_bytes[k], out->cap_bytes[k]);
            if ((t = d2h(ctx, out->bytes[k], dc.bytes[k], nb, nullptr, false))) return t;
        } else if ((t = d2h(ctx, out->col[k], dc.col[k], model_col_bytes(model, k, rows), nullptr, false))) return t;
    }
    const uint64_t ne = std::min(res->n_errors, err_cap);
    if (ne && ((t = d2h(ctx, err_line, del, ne * 8, nullptr, false)) || (t = d2h(ctx, err_code, dec, ne, nullptr, false))))
        return t;
    if ((t = d2h_wait(ctx))) return t;
    return ds == PJ_OK ? PJ_OK : fail(PJ_ERR_CAPACITY, "capacity too small (sizes needed are in the result)");
}
