// C ABI of libmans_hip.so: context, corpus handles, stream/workspace pool,
// error channel and the proof loop of the exact flat scan.
//
// The pool stands in for CommandQueuePool (CommandQueuePool.swift:27-31) and
// FlatWorkspacePool (FlatGPUSearch.swift:1070-1139): every call borrows one
// HIP stream plus its device workspace and returns them when done, so a
// context serves concurrent callers.  Streams use the default priority.
#include "mans_hip.h"
#include "mans_internal.hpp"
#include "mans_runtime.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace mans;

namespace mans {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(MANS_RESOURCE_EXHAUSTED, msg);
    return fail(MANS_EXECUTION_FAILED, msg);
}

hipError_t DevBuf::ensure(size_t need, bool inject_fail) {
    if (need <= bytes && p) return hipSuccess;
    if (inject_fail) return hipErrorOutOfMemory;
    if (p) {
        hipError_t e = hipFree(p);
        if (e != hipSuccess) return e;
        p = nullptr;
        bytes = 0;
    }
    size_t alloc = need < 256 ? 256 : need;
    hipError_t e = hipMalloc(&p, alloc);
    if (e != hipSuccess) {
        p = nullptr;
        return e;
    }
    bytes = alloc;
    return hipSuccess;
}

void DevBuf::release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
}

hipError_t PinnedBuf::ensure(size_t need) {
    if (need <= bytes && p) return hipSuccess;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    bytes = 0;
    size_t alloc = need < 256 ? 256 : need;
    hipError_t e = hipHostMalloc(&p, alloc, hipHostMallocDefault);
    if (e != hipSuccess) {
        p = nullptr;
        return e;
    }
    bytes = alloc;
    return hipSuccess;
}

void PinnedBuf::release() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    bytes = 0;
}

Slot::~Slot() {
    for (DevBuf* b : {&queries, &qidx, &cand, &gcand, &counters, &dist, &ids, &status, &heads,
                      &aux0, &aux1, &aux2, &aux3})
        b->release();
    status_h.release();
    stage_h.release();
    result_h.release();
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
}

}  // namespace mans

Slot* mans_ctx::acquire() {
    {
        std::lock_guard<std::mutex> g(mu);
        if (!free_slots.empty()) {
            Slot* s = free_slots.back();
            free_slots.pop_back();
            return s;
        }
    }
    Slot* s = new Slot();
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&s->ev0) != hipSuccess || hipEventCreate(&s->ev1) != hipSuccess) {
        delete s;
        return nullptr;
    }
    std::lock_guard<std::mutex> g(mu);
    all_slots.push_back(s);
    return s;
}

void mans_ctx::release(Slot* s) {
    std::lock_guard<std::mutex> g(mu);
    free_slots.push_back(s);
}

void mans_ctx::time_begin(Slot* s, hipStream_t st) {
    if (timing) (void)hipEventRecord(s->ev0, st);
}

void mans_ctx::time_end(Slot* s, hipStream_t st, const char* name) {
    if (!timing) return;
    (void)hipEventRecord(s->ev1, st);
    if (hipEventSynchronize(s->ev1) != hipSuccess) return;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, s->ev0, s->ev1) != hipSuccess) return;
    std::lock_guard<std::mutex> g(tmu);
    auto& t = times[name];
    t.first += ms;
    t.second += 1;
}

extern "C" {

const char* mans_last_error(void) { return g_last_error.c_str(); }

int mans_ctx_create(int device, mans_ctx** out) {
    if (!out) return fail(MANS_SEARCH_FAILED, "mans_ctx_create: out is NULL");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(MANS_DEVICE_NOT_SUPPORTED, "no HIP device present");
    if (device < 0 || device >= count)
        return fail(MANS_DEVICE_NOT_SUPPORTED, "device index out of range");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(MANS_DEVICE_NOT_SUPPORTED, "hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MANS_DEVICE_NOT_SUPPORTED,
                    std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950");
    mans_ctx* c = new mans_ctx();
    c->device = device;
    c->num_cus = prop.multiProcessorCount;
    const char* f = std::getenv("MANS_HIP_FAIL");
    if (f) {
        c->fail_alloc = std::strstr(f, "alloc") != nullptr;
        c->fail_launch = std::strstr(f, "launch") != nullptr;
    }
    DeviceGuard dg(device);
    if (hipFree(nullptr) != hipSuccess) {
        delete c;
        return fail(MANS_DEVICE_NOT_SUPPORTED, "HIP runtime initialisation failed");
    }
    // A failure here only disables mans_flat_search_device_noalloc.
    (void)noalloc_init(device);
    *out = c;
    return MANS_OK;
}

void mans_ctx_destroy(mans_ctx* ctx) {
    if (!ctx) return;
    {
        DeviceGuard dg(ctx->device);
        for (Slot* s : ctx->all_slots) {
            if (s->stream) (void)hipStreamSynchronize(s->stream);
            delete s;
        }
    }
    delete ctx;
}

int mans_corpus_upload_f32(mans_ctx* ctx, const float* rows, int64_t n, int64_t dim,
                           mans_corpus** out) {
    if (!ctx || !out) return fail(MANS_SEARCH_FAILED, "mans_corpus_upload_f32: NULL argument");
    *out = nullptr;
    if (n < 0 || dim <= 0 || (n > 0 && !rows))
        return fail(MANS_DIMENSION_MISMATCH, "mans_corpus_upload_f32: bad shape");
    if (dim > 8192)
        return fail(MANS_SEARCH_FAILED, "mans_corpus_upload_f32: dim above 8192 is not supported");
    if (n > (int64_t)0xFFFFFFFEll)
        return fail(MANS_SEARCH_FAILED, "corpus larger than the 32-bit id space");
    DeviceGuard dg(ctx->device);
    mans_corpus* c = new mans_corpus();
    c->ctx = ctx;
    c->n = n;
    c->dim = dim;
    size_t bytes = (size_t)n * (size_t)dim * sizeof(float);
    hipError_t e = c->rows.ensure(bytes ? bytes : 4, ctx->fail_alloc);
    if (e == hipSuccess) e = c->norms.ensure((size_t)(n ? n : 1) * sizeof(float), ctx->fail_alloc);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "corpus allocation");
    }
    if (n > 0) {
        e = hipMemcpy(c->rows.p, rows, bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = launch_row_norms((const float*)c->rows.p, n, (int)dim, (float*)c->norms.p, nullptr);
        if (e == hipSuccess) e = hipDeviceSynchronize();
    }
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "corpus upload");
    }
    *out = c;
    return MANS_OK;
}

// ---------------------------------------------------------------------------
// MANN v3 files (MmapIndexLoader.swift:38-196).

static uint32_t read_le32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Offsets and lengths with overflow checks, as checkedAdd / alignedOffset.
static bool add_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_add_overflow(a, b, out); }
static bool mul_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_mul_overflow(a, b, out); }
static bool align_up(int64_t v, int64_t a, int64_t* out) {
    const int64_t r = v % a;
    return r == 0 ? (*out = v, true) : add_ok(v, a - r, out);
}

// The IDMap payload as JSONDecoder decodes IDMap (IDMap.swift:88-111): a
// top-level object with externalToInternal ([String: UInt32], a JSON object),
// internalToExternal ([UInt32: String]) and nextID (UInt32) required, and
// numericToInternal ([UInt64: UInt32]) / internalToNumeric optional.
// Dictionaries whose keys are integers are encoded as flat arrays of
// alternating keys and values; an object with decimal keys is accepted too.
// Unknown keys are ignored.  The count is IDMap.count: the distinct keys of
// externalToInternal plus those of numericToInternal.
namespace {

struct JsonReader {
    const char* p;
    const char* e;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool peek(char c) {
        ws();
        return p < e && *p == c;
    }
    // A string (escapes decoded for \uXXXX below 0x80 and the one-letter
    // escapes; other code points are kept as their escape text).
    bool string(std::string* out) {
        ws();
        if (p >= e || *p != '"') return false;
        ++p;
        if (out) out->clear();
        while (p < e && *p != '"') {
            char c = *p++;
            if ((unsigned char)c < 0x20) return false;
            if (c == '\\') {
                if (p >= e) return false;
                const char x = *p++;
                switch (x) {
                case '"': case '\\': case '/': break;
                case 'b': c = '\b'; break;
                case 'f': c = '\f'; break;
                case 'n': c = '\n'; break;
                case 'r': c = '\r'; break;
                case 't': c = '\t'; break;
                case 'u': {
                    if (e - p < 4) return false;
                    unsigned v = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = p[i];
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                        else return false;
                    }
                    if (out) {
                        if (v < 0x80) out->push_back((char)v);
                        else out->append(p - 2, 6);
                    }
                    p += 4;
                    continue;
                }
                default: return false;
                }
                c = x == '"' || x == '\\' || x == '/' ? x : c;
            }
            if (out) out->push_back(c);
        }
        if (p >= e) return false;
        ++p;
        return true;
    }
    // A non-negative integer literal no larger than `max`.
    bool uint(uint64_t max, uint64_t* v) {
        ws();
        const char* s = p;
        uint64_t x = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (x > (max - d) / 10) return false;
            x = x * 10 + d;
            ++p;
        }
        if (p == s || (p - s > 1 && *s == '0')) return false;
        if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return false;
        if (v) *v = x;
        return true;
    }
    bool literal(const char* w) {
        ws();
        const size_t n = std::strlen(w);
        if ((size_t)(e - p) < n || std::memcmp(p, w, n) != 0) return false;
        p += n;
        return true;
    }
    bool value(int depth) {  // any JSON value, skipped
        if (depth > 64) return false;
        ws();
        if (p >= e) return false;
        if (*p == '"') return string(nullptr);
        if (*p == '{') {
            ++p;
            if (eat('}')) return true;
            do {
                if (!string(nullptr) || !eat(':') || !value(depth + 1)) return false;
            } while (eat(','));
            return eat('}');
        }
        if (*p == '[') {
            ++p;
            if (eat(']')) return true;
            do {
                if (!value(depth + 1)) return false;
            } while (eat(','));
            return eat(']');
        }
        if (*p == 't') return literal("true");
        if (*p == 'f') return literal("false");
        if (*p == 'n') return literal("null");
        if (*p == '-') ++p;
        const char* s = p;
        while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                         *p == '+' || *p == '-'))
            ++p;
        return p > s;
    }
    // A dictionary with integer keys (below kmax) and values of kind `val`
    // ('u': integer below vmax, 's': string): the alternating array or an
    // object with decimal keys.  keys (nullable) receives the keys.
    bool int_dict(uint64_t kmax, char val, uint64_t vmax, std::vector<uint64_t>* keys) {
        auto one_value = [&]() { return val == 's' ? string(nullptr) : uint(vmax, nullptr); };
        if (eat('[')) {
            if (eat(']')) return true;
            do {
                uint64_t k;
                if (!uint(kmax, &k) || !eat(',') || !one_value()) return false;
                if (keys) keys->push_back(k);
            } while (eat(','));
            return eat(']');
        }
        if (!eat('{')) return false;
        if (eat('}')) return true;
        std::string ks;
        do {
            if (!string(&ks) || !eat(':') || !one_value()) return false;
            JsonReader kr{ks.data(), ks.data() + ks.size()};
            uint64_t k;
            if (!kr.uint(kmax, &k) || kr.p != kr.e) return false;
            if (keys) keys->push_back(k);
        } while (eat(','));
        return eat('}');
    }
};

bool idmap_count(const uint8_t* data, int64_t len, int64_t* count) {
    JsonReader r{(const char*)data, (const char*)data + len};
    if (!r.eat('{')) return false;
    bool have_e2i = false, have_i2e = false, have_next = false;
    std::vector<std::string> ext;
    std::vector<uint64_t> numeric;
    std::string key;
    if (!r.eat('}')) {
        do {
            if (!r.string(&key) || !r.eat(':')) return false;
            if (key == "externalToInternal") {
                have_e2i = true;
                ext.clear();
                if (!r.eat('{')) return false;
                if (!r.eat('}')) {
                    std::string s;
                    do {
                        if (!r.string(&s) || !r.eat(':') || !r.uint(0xFFFFFFFFull, nullptr)) return false;
                        ext.push_back(s);
                    } while (r.eat(','));
                    if (!r.eat('}')) return false;
                }
            } else if (key == "internalToExternal") {
                have_i2e = true;
                if (!r.int_dict(0xFFFFFFFFull, 's', 0, nullptr)) return false;
            } else if (key == "nextID") {
                have_next = true;
                if (!r.uint(0xFFFFFFFFull, nullptr)) return false;
            } else if (key == "numericToInternal") {
                numeric.clear();
                if (!r.literal("null") && !r.int_dict(~0ull, 'u', 0xFFFFFFFFull, &numeric)) return false;
            } else if (key == "internalToNumeric") {
                if (!r.literal("null") && !r.int_dict(0xFFFFFFFFull, 'u', ~0ull, nullptr)) return false;
            } else if (!r.value(0)) {
                return false;
            }
        } while (r.eat(','));
        if (!r.eat('}')) return false;
    }
    r.ws();
    if (r.p != r.e || !have_e2i || !have_i2e || !have_next) return false;
    std::sort(ext.begin(), ext.end());
    std::sort(numeric.begin(), numeric.end());
    *count = (int64_t)(std::unique(ext.begin(), ext.end()) - ext.begin()) +
             (int64_t)(std::unique(numeric.begin(), numeric.end()) - numeric.begin());
    return true;
}

}  // namespace

// Validates the mapped bytes [base, base + len) as a MANN v3 file.
static int mann_parse(const uint8_t* base, int64_t len, int64_t page, mans_mann_info* info) {
    std::memset(info, 0, sizeof(*info));
    info->page_size = page;
    if (len < 4 || std::memcmp(base, "MANN", 4) != 0) return fail(MANS_CORRUPT_FILE, "Invalid file magic");
    if (len < 28) return fail(MANS_CORRUPT_FILE, "Unexpected EOF");
    info->version = read_le32(base + 4);
    if (info->version != 3)
        return fail(MANS_CORRUPT_FILE,
                    "Mmap loader requires version 3, found " + std::to_string(info->version));
    info->node_count = read_le32(base + 8);
    info->degree = read_le32(base + 12);
    info->dim = read_le32(base + 16);
    info->metric = read_le32(base + 20);
    if (info->metric > 3) return fail(MANS_CORRUPT_FILE, "Unsupported metric code");
    info->storage_type = read_le32(base + 24);
    if (info->node_count == 0) return fail(MANS_CORRUPT_FILE, "Node count must be greater than zero");
    if (info->degree == 0) return fail(MANS_CORRUPT_FILE, "Degree must be greater than zero");
    if (info->storage_type > 2)
        return fail(MANS_CORRUPT_FILE, "Unsupported storage type " + std::to_string(info->storage_type));
    if (info->dim == 0) return fail(MANS_CORRUPT_FILE, "Dimension must be greater than zero");
    const int64_t n = info->node_count, deg = info->degree, dim = info->dim;
    int64_t vbytes, edges, abytes, dbytes;
    bool ok = true;
    if (info->storage_type == 2) {
        if (dim % 8 != 0) return fail(MANS_CORRUPT_FILE, "Binary index has dim not divisible by 8");
        ok = mul_ok(n, dim / 8, &vbytes);
    } else {
        int64_t elems;
        ok = mul_ok(n, dim, &elems) && mul_ok(elems, info->storage_type == 1 ? 2 : 4, &vbytes);
    }
    ok = ok && mul_ok(n, deg, &edges) && mul_ok(edges, 4, &abytes) && mul_ok(edges, 4, &dbytes);
    int64_t voff, aoff, doff, toff, t, vlen, alen, dlen, vend, aend, dend, tend;
    ok = ok && align_up(28, page, &voff) && add_ok(voff, vbytes, &t) && align_up(t, page, &aoff) &&
         add_ok(aoff, abytes, &t) && align_up(t, page, &doff) && add_ok(doff, dbytes, &t) &&
         align_up(t, page, &toff) && align_up(vbytes, page, &vlen) && align_up(abytes, page, &alen) &&
         align_up(dbytes, page, &dlen) && add_ok(voff, vlen, &vend) && add_ok(aoff, alen, &aend) &&
         add_ok(doff, dlen, &dend) && add_ok(toff, 4, &tend);
    if (!ok) return fail(MANS_CORRUPT_FILE, "Integer overflow while computing serialized sizes");
    if (vend > len || aend > len || dend > len || tend > len)
        return fail(MANS_CORRUPT_FILE, "Mmap sections are truncated");
    const int64_t idmap = read_le32(base + toff);
    int64_t idend, epend;
    if (!add_ok(tend, idmap, &idend) || !add_ok(idend, 4, &epend) || epend > len)
        return fail(MANS_CORRUPT_FILE, "Truncated IDMap payload");
    info->entry_point = read_le32(base + idend);
    int64_t idcount = 0;
    if (!idmap_count(base + tend, idmap, &idcount))
        return fail(MANS_CORRUPT_FILE, "IDMap payload is corrupt");
    if (idcount != n) return fail(MANS_CORRUPT_FILE, "ID map size does not match node count");
    if ((int64_t)info->entry_point >= n) return fail(MANS_CORRUPT_FILE, "Entry point is out of bounds");
    info->vector_offset = voff;
    info->vector_bytes = vbytes;
    info->adjacency_offset = aoff;
    info->distance_offset = doff;
    info->trailer_offset = toff;
    info->idmap_bytes = idmap;
    return MANS_OK;
}

// A read-only mapping of a whole file, unmapped on scope exit.
struct FileMap {
    int fd = -1;
    const uint8_t* p = nullptr;
    int64_t len = 0;
    ~FileMap() {
        if (p) munmap(const_cast<uint8_t*>(p), (size_t)len);
        if (fd >= 0) close(fd);
    }
    int open_map(const char* path) {
        fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail(MANS_CORRUPT_FILE, std::string("cannot open ") + path);
        struct stat st;
        if (fstat(fd, &st) != 0) return fail(MANS_CORRUPT_FILE, "cannot stat the file");
        len = (int64_t)st.st_size;
        if (len == 0) return fail(MANS_CORRUPT_FILE, "File is too small");
        void* m = mmap(nullptr, (size_t)len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) return fail(MANS_CORRUPT_FILE, "cannot map the file");
        p = (const uint8_t*)m;
        (void)madvise(m, (size_t)len, MADV_SEQUENTIAL);
        return MANS_OK;
    }
};

static int64_t host_page_size(int64_t page) {
    if (page > 0) return page;
    const long ps = sysconf(_SC_PAGESIZE);
    return ps > 0 ? (int64_t)ps : 4096;
}

int mans_mann_inspect(const char* path, int64_t page_size, mans_mann_info* info) {
    if (!path || !info) return fail(MANS_SEARCH_FAILED, "mans_mann_inspect: NULL argument");
    FileMap fm;
    int rc = fm.open_map(path);
    if (rc != MANS_OK) return rc;
    return mann_parse(fm.p, fm.len, host_page_size(page_size), info);
}

int mans_corpus_upload_mann(mans_ctx* ctx, const char* path, int64_t page_size, mans_corpus** out,
                            uint32_t* out_metric) {
    if (!ctx || !path || !out) return fail(MANS_SEARCH_FAILED, "mans_corpus_upload_mann: NULL argument");
    *out = nullptr;
    FileMap fm;
    int rc = fm.open_map(path);
    if (rc != MANS_OK) return rc;
    mans_mann_info info;
    rc = mann_parse(fm.p, fm.len, host_page_size(page_size), &info);
    if (rc != MANS_OK) return rc;
    if (info.storage_type != 0)
        return fail(MANS_PIPELINE_UNAVAILABLE, "the device scan reads fp32 vector storage only");
    const int64_t n = info.node_count, dim = info.dim;
    if (dim > 8192) return fail(MANS_SEARCH_FAILED, "dim above 8192 is not supported");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = lease.slot->stream;
    mans_corpus* c = new mans_corpus();
    c->ctx = ctx;
    c->n = n;
    c->dim = dim;
    const size_t bytes = (size_t)info.vector_bytes;
    hipError_t e = c->rows.ensure(bytes, ctx->fail_alloc);
    if (e == hipSuccess) e = c->norms.ensure((size_t)n * sizeof(float), ctx->fail_alloc);
    // The vector section straight from the mapping, through two pinned
    // staging buffers: the host fills one while the other is copied.
    constexpr size_t kChunk = (size_t)32 << 20;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipHostMalloc(&stage[i], std::min(kChunk, bytes));
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    const uint8_t* src = fm.p + info.vector_offset;
    for (size_t off = 0, i = 0; e == hipSuccess && off < bytes; off += kChunk, ++i) {
        const size_t len = std::min(kChunk, bytes - off);
        const int b = (int)(i & 1);
        if (i >= 2) e = hipEventSynchronize(done[b]);  // the copy out of this buffer is done
        if (e != hipSuccess) break;
        std::memcpy(stage[b], src + off, len);
        e = hipMemcpyAsync((uint8_t*)c->rows.p + off, stage[b], len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(done[b], st);
    }
    if (e == hipSuccess) e = launch_row_norms((const float*)c->rows.p, n, (int)dim, (float*)c->norms.p, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    for (int i = 0; i < 2; ++i) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "MANN upload");
    }
    if (out_metric) *out_metric = info.metric;
    *out = c;
    return MANS_OK;
}

int mans_corpus_write_rows(mans_corpus* c, int64_t first_row, const float* rows, int64_t count) {
    if (!c || (count > 0 && !rows)) return fail(MANS_SEARCH_FAILED, "mans_corpus_write_rows: NULL");
    if (first_row < 0 || count < 0 || first_row + count > c->n)
        return fail(MANS_SEARCH_FAILED, "mans_corpus_write_rows: row range outside the corpus");
    if (count == 0) return MANS_OK;
    DeviceGuard dg(c->ctx->device);
    std::lock_guard<std::mutex> g(c->mu);
    float* dst = (float*)c->rows.p + first_row * c->dim;
    hipError_t e = hipMemcpy(dst, rows, (size_t)count * c->dim * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_row_norms(dst, count, (int)c->dim, (float*)c->norms.p + first_row, nullptr);
    if (e == hipSuccess && c->int8_valid)
        e = int8_refresh_rows(c, first_row, count, nullptr);
    c->bf_valid = false;  // the split parts are rebuilt on next use
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "corpus write");
    return MANS_OK;
}

int mans_corpus_invalidate(mans_corpus* c) {
    if (!c) return fail(MANS_SEARCH_FAILED, "mans_corpus_invalidate: NULL");
    std::lock_guard<std::mutex> g(c->mu);
    c->int8_valid = false;
    c->bf_valid = false;
    return MANS_OK;
}

void mans_corpus_release(mans_corpus* c) {
    if (!c) return;
    DeviceGuard dg(c->ctx->device);
    (void)hipDeviceSynchronize();
    delete c;
}

int64_t mans_corpus_count(const mans_corpus* c) { return c ? c->n : -1; }
int64_t mans_corpus_dim(const mans_corpus* c) { return c ? c->dim : -1; }

int mans_timing_enable(mans_ctx* ctx, int enable) {
    if (!ctx) return fail(MANS_SEARCH_FAILED, "NULL context");
    ctx->timing = enable != 0;
    return MANS_OK;
}

int mans_timing_read(mans_ctx* ctx, const char* kernel, double* total_ms, int64_t* launches) {
    if (!ctx || !kernel) return fail(MANS_SEARCH_FAILED, "NULL argument");
    std::lock_guard<std::mutex> g(ctx->tmu);
    auto it = ctx->times.find(kernel);
    if (total_ms) *total_ms = it == ctx->times.end() ? 0.0 : it->second.first;
    if (launches) *launches = it == ctx->times.end() ? 0 : it->second.second;
    return MANS_OK;
}

int mans_timing_reset(mans_ctx* ctx) {
    if (!ctx) return fail(MANS_SEARCH_FAILED, "NULL context");
    std::lock_guard<std::mutex> g(ctx->tmu);
    ctx->times.clear();
    return MANS_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Exact flat scan driver.
// ---------------------------------------------------------------------------

namespace mans {

static int pow2_ceil(int64_t x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// Sizes the slot's flat-scan buffers for one launch.  The merge counters
// are zeroed when the buffer is new or a launch failed; a completed launch
// leaves them zero.
hipError_t prepare_flat_buffers(mans_ctx* ctx, Slot* slot, const FlatPlan& p, int64_t nq,
                                hipStream_t st, FlatBuffers* out) {
    size_t cnt_bytes = (size_t)nq * (size_t)(p.ngroups + 1) * sizeof(uint32_t);
    bool fresh = cnt_bytes > slot->counters.bytes || !slot->counters.p;
    hipError_t e = slot->cand.ensure((size_t)nq * p.nblk * p.kc * sizeof(uint64_t), ctx->fail_alloc);
    if (e == hipSuccess)
        e = slot->gcand.ensure((size_t)nq * p.ngroups * p.kc * sizeof(uint64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->counters.ensure(cnt_bytes, ctx->fail_alloc);
    if (e == hipSuccess) e = slot->status.ensure((size_t)nq, ctx->fail_alloc);
    if (e != hipSuccess) return e;
    if (p.fast) {
        e = slot->heads.ensure((size_t)nq * p.nblk * sizeof(uint64_t), ctx->fail_alloc);
        if (e != hipSuccess) return e;
        out->heads = (uint64_t*)slot->heads.p;
    }
    if (fresh || slot->counters_dirty) {
        e = hipMemsetAsync(slot->counters.p, 0, slot->counters.bytes, st);
        if (e != hipSuccess) return e;
        slot->counters_dirty = false;
    }
    out->cand = (uint64_t*)slot->cand.p;
    out->gcand = (uint64_t*)slot->gcand.p;
    out->counters = (uint32_t*)slot->counters.p;
    out->status = (uint8_t*)slot->status.p;
    return hipSuccess;
}

hipError_t fill_empty(float* dist, uint32_t* ids, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipError_t e = hipMemsetD32Async((hipDeviceptr_t)dist, 0x7F7FFFFF, (size_t)count, s);
    if (e == hipSuccess) e = hipMemsetD32Async((hipDeviceptr_t)ids, 0xFFFFFFFF, (size_t)count, s);
    return e;
}

// Host <-> device copies through the slot's pinned staging buffer (a
// pageable copy costs an extra driver-side bounce).
hipError_t stage_to_device(Slot* s, void* dst, const void* src, size_t bytes) {
    hipError_t e = s->stage_h.ensure(bytes);
    if (e != hipSuccess) return e;
    std::memcpy(s->stage_h.p, src, bytes);
    return hipMemcpyAsync(dst, s->stage_h.p, bytes, hipMemcpyHostToDevice, s->stream);
}

hipError_t stage_from_device(Slot* s, void* dst0, const void* src0, size_t b0, void* dst1,
                             const void* src1, size_t b1) {
    // The previous staging upload may still be in flight on the stream.
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e == hipSuccess) e = s->stage_h.ensure(b0 + b1);
    if (e == hipSuccess)
        e = hipMemcpyAsync(s->stage_h.p, src0, b0, hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess && b1)
        e = hipMemcpyAsync((char*)s->stage_h.p + b0, src1, b1, hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return e;
    std::memcpy(dst0, s->stage_h.p, b0);
    if (b1) std::memcpy(dst1, (char*)s->stage_h.p + b0, b1);
    return hipSuccess;
}

// Runs the flat scan for queries already in device memory.  The proof loop
// (kc x4 per round, exact keys past kc = 1024) mirrors the budget growth of
// BoundedExactScan.swift:96-121.
// MANS_BF16_SPLIT=0 keeps batches on the fp32 contraction.
static bool bf16_split_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MANS_BF16_SPLIT");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Builds the split-bf16 parts of the rows on first use (and after writes).
static int bf16_split_ensure(mans_ctx* ctx, const mans_corpus* cc, hipStream_t st) {
    mans_corpus* c = const_cast<mans_corpus*>(cc);
    std::lock_guard<std::mutex> g(c->mu);
    if (c->bf_valid) return MANS_OK;
    if (c->dim % 16 != 0) {
        c->bf_valid = true;
        c->bf_ok = false;
        return MANS_OK;
    }
    hipError_t e = c->bf_hi.ensure((size_t)c->n * c->dim * sizeof(uint16_t), ctx->fail_alloc);
    if (e == hipSuccess) e = c->bf_rec.ensure((size_t)c->n * 8 * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = c->bf_flag.ensure(sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = hipMemsetAsync(c->bf_flag.p, 0, sizeof(uint32_t), st);
    if (e == hipSuccess)
        e = launch_split_rows((const float*)c->rows.p, (const float*)c->norms.p, c->n, (int)c->dim,
                              (uint16_t*)c->bf_hi.p, (float*)c->bf_rec.p, (uint32_t*)c->bf_flag.p, st);
    uint32_t flag = 1;
    if (e == hipSuccess)
        e = hipMemcpyAsync(&flag, c->bf_flag.p, sizeof(uint32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "split-bf16 rows");
    c->bf_valid = true;
    c->bf_ok = flag == 0;
    return MANS_OK;
}

static int flat_search_chunk(mans_ctx* ctx, const mans_corpus* c, const float* d_q, int64_t nq,
                             int64_t k, uint32_t metric, float* d_dist, uint32_t* d_ids,
                             hipStream_t st, Slot* slot, float* h_dist, uint32_t* h_ids);

// Queries go through in chunks so the grid's y extent and the candidate
// workspace stay bounded.
int flat_search_run(mans_ctx* ctx, const mans_corpus* c, const float* d_q, int64_t nq, int64_t k,
                    uint32_t metric, float* d_dist, uint32_t* d_ids, hipStream_t st, Slot* slot,
                    float* h_dist, uint32_t* h_ids) {
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "flat scan does not support this metric");
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    const int64_t chunk = 16384;
    for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
        int64_t m = std::min(chunk, nq - q0);
        int rc = flat_search_chunk(ctx, c, d_q + q0 * c->dim, m, k, metric, d_dist + q0 * k,
                                   d_ids + q0 * k, st, slot, h_dist ? h_dist + q0 * k : nullptr,
                                   h_ids ? h_ids + q0 * k : nullptr);
        if (rc != MANS_OK) return rc;
    }
    return MANS_OK;
}

static int flat_search_chunk(mans_ctx* ctx, const mans_corpus* c, const float* d_q, int64_t nq,
                             int64_t k, uint32_t metric, float* d_dist, uint32_t* d_ids,
                             hipStream_t st, Slot* slot, float* h_dist, uint32_t* h_ids) {
    const int64_t n = c->n;
    const int dim = (int)c->dim;
    const int kstride = (int)k;
    const size_t obytes = (size_t)nq * k * sizeof(float);
    if (n == 0) {
        hipError_t e = fill_empty(d_dist, d_ids, nq * k, st);
        if (e == hipSuccess && h_dist)
            e = hipMemcpyAsync(h_dist, d_dist, obytes, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess && h_ids)
            e = hipMemcpyAsync(h_ids, d_ids, obytes, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e == hipSuccess ? MANS_OK : hip_fail(e, "fill");
    }
    const int keff = (int)std::min<int64_t>(std::min<int64_t>(k, MANS_MAX_TOP_K), n);
    int kc = pow2_ceil(std::max(32, 2 * keff));
    // The float4 path needs 16-byte aligned rows and queries.
    bool exact = flat_nch_for_dim(dim) == 0 || (reinterpret_cast<uintptr_t>(d_q) & 15u) != 0;
    std::vector<uint32_t> pending;  // empty = all queries
    int64_t npend = nq;
    for (;;) {
        if (exact) kc = pow2_ceil(std::max(32, keff));
        hipError_t e = hipSuccess;
        GemmPlan gp;
        if (pending.empty() && !exact && plan_gemm(n, dim, npend, kc, &gp)) {
            // First round of a batch: MFMA contraction + per-query merge,
            // on split-bf16 MFMA when the corpus allows it, else fp32 MFMA.
            // The split path's keys are looser (the rows keep only their
            // high parts): it keeps kGemmMaxKc candidates.
            const bool bf = bf16_split_enabled() && bf16_split_ensure(ctx, c, st) == MANS_OK && c->bf_ok;
            if (bf && kc < kGemmMaxKc) {
                kc = kGemmMaxKc;
                (void)plan_gemm(n, dim, npend, kc, &gp);
            }
            if (bf) gp.lps = 4;
            const size_t lbytes = gemm_lists_bytes(gp, npend);
            e = slot->cand.ensure(lbytes + (size_t)npend * sizeof(uint64_t), ctx->fail_alloc);
            if (e == hipSuccess) e = slot->status.ensure((size_t)npend, ctx->fail_alloc);
            if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
            if (e == hipSuccess && bf)
                e = slot->qsplit.ensure((size_t)npend * dim * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess && bf)
                e = slot->qbad.ensure((size_t)npend * sizeof(uint32_t), ctx->fail_alloc);
            if (e != hipSuccess) return hip_fail(e, "flat scan workspace");
            FlatBuffers fb;
            fb.out_dist = d_dist;
            fb.out_ids = d_ids;
            // The proof status goes straight to pinned host memory (read
            // after the round's one synchronisation, no copy).
            fb.status = (uint8_t*)slot->status_h.p;
            uint64_t* lists = (uint64_t*)slot->cand.p;
            uint64_t* qbound = bf ? lists + lbytes / sizeof(uint64_t) : nullptr;
            const uint32_t* qbad = bf ? (const uint32_t*)slot->qbad.p : nullptr;
            const float* rows = (const float*)c->rows.p;
            const float* norms = (const float*)c->norms.p;
            if (bf) {
                uint32_t* qs = (uint32_t*)slot->qsplit.p;
                const uint16_t* hi = (const uint16_t*)c->bf_hi.p;
                const float* rec = (const float*)c->bf_rec.p;
                ctx->time_begin(slot, st);
                e = hipMemsetAsync(slot->qbad.p, 0, (size_t)npend * sizeof(uint32_t), st);
                if (e == hipSuccess)
                    e = launch_split_queries(d_q, npend, dim, qs, (uint32_t*)slot->qbad.p, st);
                if (e == hipSuccess)
                    e = launch_flat_bf2(gp, true, hi, rec, n, dim, qs, d_q, npend, (int)metric,
                                        nullptr, lists, nullptr, st);
                if (e == hipSuccess)
                    e = launch_bf2_bounds(gp, npend, keff, lists, rows, norms, dim, d_q,
                                          (int)metric, qbound, st);
                ctx->time_end(slot, st, "flat_bound");
                ctx->time_begin(slot, st);
                if (e == hipSuccess)
                    e = launch_flat_bf2(gp, false, hi, rec, n, dim, qs, d_q, npend, (int)metric,
                                        qbound, lists, (uint32_t*)slot->qbad.p, st);
                ctx->time_end(slot, st, "flat_gemm");
            } else {
                ctx->time_begin(slot, st);
                e = launch_flat_gemm(gp, rows, norms, n, dim, d_q, npend, (int)metric, lists, st);
                ctx->time_end(slot, st, "flat_gemm");
            }
            ctx->time_begin(slot, st);
            if (e == hipSuccess)
                e = launch_flat_gemm_merge(gp, rows, norms, n, dim, d_q, npend, (int)metric, lists,
                                           qbound, qbad, fb, keff, kstride, st);
            ctx->time_end(slot, st, "flat_merge");
        } else {
            FlatPlan p = plan_flat(n, npend, kc);
            const uint32_t* d_qidx = nullptr;
            if (!pending.empty()) {
                e = slot->qidx.ensure(pending.size() * sizeof(uint32_t), ctx->fail_alloc);
                if (e == hipSuccess)
                    e = hipMemcpyAsync(slot->qidx.p, pending.data(),
                                       pending.size() * sizeof(uint32_t), hipMemcpyHostToDevice, st);
                d_qidx = (const uint32_t*)slot->qidx.p;
            }
            FlatBuffers fb;
            if (e == hipSuccess) e = prepare_flat_buffers(ctx, slot, p, npend, st, &fb);
            if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
            if (e != hipSuccess) return hip_fail(e, "flat scan workspace");
            fb.out_dist = d_dist;
            fb.out_ids = d_ids;
            fb.status = (uint8_t*)slot->status_h.p;
            ctx->time_begin(slot, st);
            e = launch_flat_search(p, exact, (const float*)c->rows.p, (const float*)c->norms.p, n,
                                   dim, d_q, d_qidx, npend, (int)metric, fb, keff, kstride, st);
            ctx->time_end(slot, st, "flat_scan");
        }
        // Results (when the caller wants them on the host) come back with
        // the round's one synchronisation; the proof status is already in
        // pinned host memory.
        if (e == hipSuccess && h_dist)
            e = hipMemcpyAsync(h_dist, d_dist, obytes, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess && h_ids)
            e = hipMemcpyAsync(h_ids, d_ids, obytes, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "flat scan");
        }
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        std::vector<uint32_t> next;
        for (int64_t i = 0; i < npend; ++i)
            if (sh[i]) next.push_back(pending.empty() ? (uint32_t)i : pending[i]);
        if (next.empty()) return MANS_OK;
        if (exact) return fail(MANS_SEARCH_FAILED, "exact round failed its own proof");
        pending.swap(next);
        npend = (int64_t)pending.size();
        kc *= 4;
        if (kc > 1024) exact = true;
        ctx->proof_retries += npend;
    }
}

}  // namespace mans

extern "C" {

int mans_flat_search_device(mans_ctx* ctx, const mans_corpus* c, const float* d_queries,
                            int64_t nq, int64_t k, uint32_t metric, float* d_out_dist,
                            uint32_t* d_out_ids, void* stream) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq > 0 && k > 0 && (!d_queries || !d_out_dist || !d_out_ids))
        return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = stream ? (hipStream_t)stream : lease.slot->stream;
    return flat_search_run(ctx, c, d_queries, nq, k, metric, d_out_dist, d_out_ids, st, lease.slot,
                           nullptr, nullptr);
}

int mans_flat_search(mans_ctx* ctx, const mans_corpus* c, const float* queries, int64_t nq,
                     int64_t k, uint32_t metric, float* out_dist, uint32_t* out_ids) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (!queries || !out_dist || !out_ids) return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    Slot* s = lease.slot;
    if (!s) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    size_t qbytes = (size_t)nq * c->dim * sizeof(float);
    size_t obytes = (size_t)nq * k * sizeof(float);
    hipError_t e = s->queries.ensure(qbytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->dist.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->ids.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->result_h.ensure(2 * obytes);
    if (e == hipSuccess) e = stage_to_device(s, s->queries.p, queries, qbytes);
    if (e != hipSuccess) return hip_fail(e, "flat scan staging");
    // The kernels write the results straight into pinned host memory
    // (device-accessible): no copies back, one synchronisation.
    float* hd = (float*)s->result_h.p;
    uint32_t* hi = (uint32_t*)((char*)s->result_h.p + obytes);
    int rc = flat_search_run(ctx, c, (const float*)s->queries.p, nq, k, metric, hd, hi, s->stream,
                             s, nullptr, nullptr);
    if (rc != MANS_OK) return rc;
    std::memcpy(out_dist, hd, obytes);
    std::memcpy(out_ids, hi, obytes);
    return MANS_OK;
}

}  // extern "C"
