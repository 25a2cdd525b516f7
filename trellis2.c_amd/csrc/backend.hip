// backend.hip - trellis_sparse_backend_ops implementation for MI355X (gfx950).
//
// Host side of the drop-in backend: argument and status contract of the
// reference CPU backend (src/ops/sparse/trellis_sparse_cpu.c), device buffer
// pool, weight cache keyed by host pointer (the Vulkan backend's contract,
// src/ops/sparse/trellis_sparse_vulkan.c:1019-1052), device-resident C2S maps
// (vtable slots 18-25, src/ops/sparse/trellis_sparse_backend.h:119-182) and
// stage timing with HIP events on the backend's stream.
//
// Threading: one backend instance is single-threaded, like the reference
// backends (trellis_sparse_vulkan.c:163-187); separate instances are
// independent.  Every call enqueues on the instance's own stream; calls that
// hand data back to the host (download_*, build_c2s_map*, n_out) synchronise.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>

#include "tsh_internal.h"

namespace tsh {

struct WeightKey {
    const void * ptr;
    size_t count;
    int layout;
    int ci, co;
    bool operator==(const WeightKey & o) const {
        return ptr == o.ptr && count == o.count && layout == o.layout && ci == o.ci && co == o.co;
    }
};
struct WeightKeyHash {
    size_t operator()(const WeightKey & k) const {
        return std::hash<const void *>()(k.ptr) ^ (k.count * 0x9e3779b97f4a7c15ull) ^ ((size_t) k.layout << 56) ^
               ((size_t) k.ci << 20) ^ (size_t) k.co;
    }
};

enum WeightLayout : int {
    kLayoutConvF32 = 1,   // fp32 [27][ci][co]
    kLayoutConvMfma = 2,  // storage type [27][ci/8][co][8]
    kLayoutLinearT = 3,   // fp32 [ci][co]
    kLayoutVector = 4,    // fp32 [count]
    kLayoutConvMfmaGrouped = 5,  // kLayoutConvMfma with the compacted kernels' column grouping
    kLayoutLinearMfma = 6,       // storage type [ci/8][co][8], linear_mfma_group column grouping
    kLayoutMlp0 = 7,             // as kLayoutLinearMfma, the fused MLP's first GEMM grouping
    kLayoutMlp2 = 8,             // as kLayoutLinearMfma, the fused MLP's second GEMM grouping
    kLayoutLinear16 = 9          // storage type [co][ci] (narrow MFMA linear)
};

struct StageMark {
    hipEvent_t a = nullptr, b = nullptr;
    int stage = 0;
};

struct IntoScratch;

struct Backend {
    trellis_sparse_backend base;
    int device = 0;
    int cus = 0;  // compute units of the device
    hipStream_t stream = nullptr;
    trellis_sparse_hip_policy policy{};
    std::string last_error;
    // Pool: size class -> free device blocks.
    std::map<size_t, std::vector<void *>> free_blocks;
    size_t pooled_bytes = 0;
    // Forced allocation failures (tests of the out-of-memory paths): device
    // allocation attempts fail_after .. fail_after + fail_count - 1 (counted
    // from 0 since the hook was set) report hipErrorOutOfMemory without
    // calling hipMalloc.  fail_after < 0: off.
    int64_t fail_after = -1;
    int64_t fail_count = 0;
    int64_t alloc_attempts = 0;
    // Device address of this device's copy of `scratch` (the allocation-free
    // subdivide's working memory), or null when it could not be resolved.
    IntoScratch * into = nullptr;  // build_c2s_map_into's scratch on this backend's device
    // The platform GEMM library's handle, plans and workspace for the wide
    // linears (created on first use; the workspace goes with trim(FREE_BUFFERS)).
    LinearLt * lt = nullptr;
    DevMem lt_ws;
    // Weight cache.
    std::unordered_map<WeightKey, DevMem, WeightKeyHash> weights;
    std::vector<DevMem> transient;  // uncached weights of the current call
    // Device C2S maps (valid until destroy).
    std::vector<trellis_sparse_c2s_device_map *> maps;
    // Pinned host staging for downloads into caller-owned pageable arrays
    // (grown on demand; released by trim(FREE_BUFFERS) and destroy).
    void * pinned = nullptr;
    size_t pinned_bytes = 0;
    // Pinned words for small device-to-host reads (child and face counts),
    // and the event the host spins on for them (allocated at creation).
    int32_t * host_words = nullptr;
    hipEvent_t words_ready = nullptr;
    // Timing.
    bool profiling = false;
    std::vector<StageMark> pending;
    std::vector<hipEvent_t> spare_events;
    trellis_sparse_hip_stage_times times{};
    hipEvent_t user_events[16] = {};
    StageMark open[TRELLIS_SPARSE_HIP_STAGE_COUNT];
};

// Working memory of trellis_sparse_hip_build_c2s_map_into, which allocates
// nothing: per-parent child counts, their exclusive scan, the scan total and
// the scan's tile sums, for at most kIntoMaxParents parents.  Each device
// holds its own copy until the process ends.  Host code uses the device
// address from hipGetSymbolAddress (resolved once per device at backend
// creation), never the array's name: in host code the name is a host-side
// stand-in, not a device address.
constexpr int64_t kIntoMaxParents = int64_t(1) << 20;
constexpr size_t kIntoCounts = 0;                                        // int32 [kIntoMaxParents]
constexpr size_t kIntoOffsets = kIntoCounts + 4 * kIntoMaxParents;       // int32 [kIntoMaxParents]
constexpr size_t kIntoTotal = kIntoOffsets + 4 * kIntoMaxParents;        // int32, own 256-byte line
constexpr size_t kIntoSums = kIntoTotal + 256;                           // scan tile sums
constexpr size_t kIntoScratchBytes = kIntoSums + 16384;
static __device__ __align__(256) unsigned char scratch[kIntoScratchBytes];

// Per device: the address of its copy of `scratch`, and the lock and event
// that order calls on that device (each call waits, on its own stream, for
// the previous call's last kernel, which still reads the scratch after the
// previous call returned).
struct IntoScratch {
    unsigned char * addr = nullptr;
    hipEvent_t done = nullptr;
    std::mutex mu;
};

// Resolves this device's copy of `scratch` and creates its event, once per
// device (the caller has made `device` current).  Returns null on failure.
IntoScratch * scratch_for(int device) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static IntoScratch dev[kMaxDevices];
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    IntoScratch & d = dev[device];
    if (d.addr == nullptr) {
        void * p = nullptr;
        hipEvent_t e = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr ||
            hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            (void) hipGetLastError();
            return nullptr;
        }
        d.done = e;
        d.addr = (unsigned char *) p;
    }
    return &d;
}

namespace {

Backend * as_backend(trellis_sparse_backend * b) { return reinterpret_cast<Backend *>(b); }
const Backend * as_backend(const trellis_sparse_backend * b) { return reinterpret_cast<const Backend *>(b); }

trellis_status fail(Backend * be, trellis_status st, const char * what) {
    if (be != nullptr) be->last_error = what;
    return st;
}

trellis_status hip_status(Backend * be, hipError_t err, const char * where) {
    if (err == hipSuccess) return TRELLIS_STATUS_OK;
    if (be != nullptr) {
        be->last_error = std::string(where) + ": " + hipGetErrorString(err);
    }
    (void) hipGetLastError();
    return err == hipErrorOutOfMemory ? TRELLIS_STATUS_OUT_OF_MEMORY : TRELLIS_STATUS_ERROR;
}

#define TSH_TRY(be, expr)                                            \
    do {                                                             \
        const hipError_t tsh_err_ = (expr);                          \
        if (tsh_err_ != hipSuccess) return hip_status(be, tsh_err_, #expr); \
    } while (0)

size_t size_class(size_t bytes) {
    if (bytes <= 4096) return 4096;
    // Four classes per power of two (at most 25% slack).
    size_t p = 4096;
    while (p * 2 < bytes) p *= 2;
    const size_t step = p / 4;
    return (bytes + step - 1) / step * step;
}

hipError_t device_malloc(Backend * be, void ** p, size_t bytes) {
    *p = nullptr;
    if (be->fail_after >= 0) {
        const int64_t attempt = be->alloc_attempts++;
        if (attempt >= be->fail_after && attempt - be->fail_after < be->fail_count) return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

trellis_status dev_alloc(Backend * be, size_t bytes, DevMem * out) {
    out->ptr = nullptr;
    out->bytes = 0;
    if (bytes == 0) return TRELLIS_STATUS_OK;
    const size_t cls = size_class(bytes);
    auto it = be->free_blocks.find(cls);
    if (it != be->free_blocks.end() && !it->second.empty()) {
        out->ptr = it->second.back();
        it->second.pop_back();
        be->pooled_bytes -= cls;
        out->bytes = cls;
        return TRELLIS_STATUS_OK;
    }
    void * p = nullptr;
    hipError_t err = device_malloc(be, &p, cls);
    if (err == hipErrorOutOfMemory && be->pooled_bytes > 0) {
        // Release cached blocks and retry once.
        (void) hipGetLastError();
        (void) hipStreamSynchronize(be->stream);
        for (auto & kv : be->free_blocks) {
            for (void * q : kv.second) (void) hipFree(q);
            kv.second.clear();
        }
        be->pooled_bytes = 0;
        err = device_malloc(be, &p, cls);
    }
    if (err != hipSuccess) {
        return hip_status(be, err, "hipMalloc");
    }
    out->ptr = p;
    out->bytes = cls;
    return TRELLIS_STATUS_OK;
}

// Returns a block to the pool.  Work already queued on the backend stream may
// still use it; any later user is queued behind that work on the same stream.
void dev_release(Backend * be, DevMem * m) {
    if (m == nullptr || m->ptr == nullptr) return;
    be->free_blocks[m->bytes].push_back(m->ptr);
    be->pooled_bytes += m->bytes;
    m->ptr = nullptr;
    m->bytes = 0;
}

void select_device(Backend * be) { (void) hipSetDevice(be->device); }

// memcpy split over up to 8 host threads (at least 2 MiB each): copying into
// freshly allocated pageable memory is bound by first-touch page faults,
// which threads take in parallel.
void parallel_copy(void * dst, const void * src, size_t bytes) {
    constexpr size_t kMinChunk = (size_t) 2 << 20;
    const size_t parts = std::min<size_t>(8, std::max<size_t>(1, bytes / kMinChunk));
    if (parts <= 1) {
        memcpy(dst, src, bytes);
        return;
    }
    const size_t chunk = (bytes + parts - 1) / parts;
    std::vector<std::thread> pool;
    for (size_t i = 1; i < parts; ++i) {
        const size_t off = i * chunk, len = std::min(chunk, bytes - off);
        pool.emplace_back([=] { memcpy((char *) dst + off, (const char *) src + off, len); });
    }
    memcpy(dst, src, chunk);
    for (auto & th : pool) th.join();
}

// Pinned staging of at least `bytes` (the stream has no transfer pending on
// the old buffer when this is called: every user synchronizes before
// returning).
trellis_status pinned_reserve(Backend * be, size_t bytes) {
    if (bytes <= be->pinned_bytes) return TRELLIS_STATUS_OK;
    if (be->pinned != nullptr) (void) hipHostFree(be->pinned);
    be->pinned = nullptr;
    be->pinned_bytes = 0;
    const size_t want = std::max<size_t>(bytes, (size_t) 1 << 20);
    void * p = nullptr;
    if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) {
        (void) hipGetLastError();
        return fail(be, TRELLIS_STATUS_OUT_OF_MEMORY, "pinned staging buffer");
    }
    be->pinned = p;
    be->pinned_bytes = want;
    return TRELLIS_STATUS_OK;
}

// Reads up to kHostWords int32 values from device memory (one or two source
// ranges) into host variables, through the backend's pinned words: the
// copies write host memory directly, and the host polls an event for up to
// kSpinMicros, so it resumes within microseconds of a short wait, where a
// blocking stream synchronisation and a pageable destination cost tens of
// microseconds; longer waits (work still queued ahead of the copy) block in
// hipEventSynchronize instead of spinning.  The queue is drained up to the
// copy, as hipStreamSynchronize would.
constexpr int kSpinMicros = 50;
constexpr int kHostWords = 16;
hipError_t read_words(Backend * be, hipStream_t s, int32_t * dst0, const void * src0, int count0,
                      int32_t * dst1 = nullptr, const void * src1 = nullptr, int count1 = 0) {
    if (be->host_words == nullptr || be->words_ready == nullptr || count0 + count1 > kHostWords) {
        hipError_t err = hipMemcpyAsync(dst0, src0, (size_t) count0 * 4, hipMemcpyDeviceToHost, s);
        if (err == hipSuccess && count1 > 0) err = hipMemcpyAsync(dst1, src1, (size_t) count1 * 4, hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);
        return err;
    }
    hipError_t err = hipMemcpyAsync(be->host_words, src0, (size_t) count0 * 4, hipMemcpyDeviceToHost, s);
    if (err == hipSuccess && count1 > 0) {
        err = hipMemcpyAsync(be->host_words + count0, src1, (size_t) count1 * 4, hipMemcpyDeviceToHost, s);
    }
    if (err == hipSuccess) err = hipEventRecord(be->words_ready, s);
    if (err != hipSuccess) return err;
    const auto spin_end = std::chrono::steady_clock::now() + std::chrono::microseconds(kSpinMicros);
    while ((err = hipEventQuery(be->words_ready)) == hipErrorNotReady) {
        if (std::chrono::steady_clock::now() >= spin_end) {
            err = hipEventSynchronize(be->words_ready);
            break;
        }
    }
    (void) hipGetLastError();  // the not-ready polls are not errors
    if (err != hipSuccess) return err;
    const volatile int32_t * w = be->host_words;
    for (int i = 0; i < count0; ++i) dst0[i] = w[i];
    for (int i = 0; i < count1; ++i) dst1[i] = w[count0 + i];
    return hipSuccess;
}

// ---- stage timing -----------------------------------------------------------
hipEvent_t take_event(Backend * be) {
    if (!be->spare_events.empty()) {
        hipEvent_t e = be->spare_events.back();
        be->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void) hipGetLastError();
        return nullptr;
    }
    return e;
}

void stage_begin(Backend * be, int stage) {
    if (!be->profiling) return;
    StageMark & m = be->open[stage];
    m.stage = stage;
    m.a = take_event(be);
    m.b = take_event(be);
    if (m.a != nullptr) (void) hipEventRecord(m.a, be->stream);
}

void stage_end(Backend * be, int stage) {
    if (!be->profiling) return;
    StageMark m = be->open[stage];
    be->open[stage] = StageMark{};
    if (m.a == nullptr || m.b == nullptr) return;
    (void) hipEventRecord(m.b, be->stream);
    be->pending.push_back(m);
}

// ---- buffers ---------------------------------------------------------------
trellis_status new_buffer(Backend * be, size_t count, int dtype, trellis_sparse_buffer ** out) {
    const size_t elem = dtype < 0 ? 4u : dtype_bytes(dtype);
    if (count > SIZE_MAX / elem) return fail(be, TRELLIS_STATUS_OUT_OF_MEMORY, "buffer size overflow");
    auto * b = (trellis_sparse_buffer *) calloc(1, sizeof(trellis_sparse_buffer));
    if (b == nullptr) return fail(be, TRELLIS_STATUS_OUT_OF_MEMORY, "host allocation");
    DevMem m;
    const trellis_status st = dev_alloc(be, count * elem, &m);
    if (st != TRELLIS_STATUS_OK) {
        free(b);
        return st;
    }
    b->ptr = m.ptr;
    b->count = count;
    b->bytes = count * elem;
    b->cap = m.bytes;
    b->dtype = dtype;
    *out = b;
    return TRELLIS_STATUS_OK;
}

bool float_buffer_ok(const Backend * be, const trellis_sparse_buffer * b, size_t need) {
    return b != nullptr && b->dtype == be->policy.compute_dtype && b->count >= need && (need == 0 || b->ptr != nullptr);
}

// Uploads host bytes to a device block through the backend stream and waits,
// so the caller's memory may be reused on return.
trellis_status upload_bytes(Backend * be, const void * src, size_t bytes, DevMem * out) {
    trellis_status st = dev_alloc(be, bytes, out);
    if (st != TRELLIS_STATUS_OK) return st;
    if (bytes == 0) return TRELLIS_STATUS_OK;
    TSH_TRY(be, hipMemcpyAsync(out->ptr, src, bytes, hipMemcpyHostToDevice, be->stream));
    TSH_TRY(be, hipStreamSynchronize(be->stream));
    return TRELLIS_STATUS_OK;
}

// ---- weight / vector cache ---------------------------------------------------
trellis_status get_weight(Backend * be, const float * host, size_t count, int layout, int ci, int co,
                          const void ** dev_out) {
    *dev_out = nullptr;
    if (host == nullptr) return TRELLIS_STATUS_OK;
    const WeightKey key{host, count, layout, ci, co};
    if (be->policy.cache_weights) {
        auto it = be->weights.find(key);
        if (it != be->weights.end()) {
            *dev_out = it->second.ptr;
            return TRELLIS_STATUS_OK;
        }
    }
    std::vector<unsigned char> staged;
    const int dt = be->policy.compute_dtype;
    switch (layout) {
        case kLayoutConvF32: {  // [co][27][ci] -> [27][ci][co]
            staged.resize((size_t) 27 * ci * co * sizeof(float));
            float * w = (float *) staged.data();
            for (int o = 0; o < co; ++o)
                for (int k = 0; k < 27; ++k)
                    for (int c = 0; c < ci; ++c)
                        w[((size_t) k * ci + c) * co + o] = host[((size_t) o * 27 + k) * ci + c];
            break;
        }
        case kLayoutConvMfma:  // [co][27][ci] -> [27][ci/8][co][8] in the storage type
        case kLayoutConvMfmaGrouped: {
            const size_t elems = (size_t) 27 * ci * co;
            staged.resize(elems * 2);
            uint16_t * w = (uint16_t *) staged.data();
            const int ci8 = ci / 8;
            const int g = conv_stream_group(ci, co), wn = 16 * g;
            for (int o = 0; o < co; ++o) {
                // Packed column of channel o.
                const int pos = layout == kLayoutConvMfma ? o : (o / wn) * wn + (o % g) * 16 + (o % wn) / g;
                for (int k = 0; k < 27; ++k)
                    for (int c = 0; c < ci; ++c) {
                        const float v = host[((size_t) o * 27 + k) * ci + c];
                        uint16_t h;
                        if (dt == kBF16) {
                            h = f32_to_bf16(v);
                        } else {
                            const _Float16 f = (_Float16) v;
                            memcpy(&h, &f, 2);
                        }
                        w[((((size_t) k * ci8 + c / 8) * co + pos) * 8) + (c & 7)] = h;
                    }
            }
            break;
        }
        case kLayoutLinearMfma:  // [co][ci] -> [ci/8][co][8] in the storage type, grouped columns
        case kLayoutMlp0:
        case kLayoutMlp2: {
            staged.resize((size_t) ci * co * 2);
            uint16_t * w = (uint16_t *) staged.data();
            int g = linear_mfma_group(co);
            if (layout != kLayoutLinearMfma) {
                int g0 = 1, g2 = 1;
                convnext_mlp_groups(layout == kLayoutMlp0 ? ci : co, &g0, &g2);
                g = layout == kLayoutMlp0 ? g0 : g2;
            }
            const int wn = 16 * g;
            for (int o = 0; o < co; ++o) {
                const int pos = (o / wn) * wn + (o % g) * 16 + (o % wn) / g;
                for (int c = 0; c < ci; ++c) {
                    const float v = host[(size_t) o * ci + c];
                    uint16_t h;
                    if (dt == kBF16) {
                        h = f32_to_bf16(v);
                    } else {
                        const _Float16 f = (_Float16) v;
                        memcpy(&h, &f, 2);
                    }
                    w[(((size_t) (c / 8) * co + pos) * 8) + (c & 7)] = h;
                }
            }
            break;
        }
        case kLayoutLinear16: {  // [co][ci] in the storage type
            staged.resize((size_t) ci * co * 2);
            uint16_t * w = (uint16_t *) staged.data();
            for (size_t i = 0; i < (size_t) ci * co; ++i) {
                if (dt == kBF16) {
                    w[i] = f32_to_bf16(host[i]);
                } else {
                    const _Float16 f = (_Float16) host[i];
                    memcpy(&w[i], &f, 2);
                }
            }
            break;
        }
        case kLayoutLinearT: {  // [co][ci] -> [ci][co]
            staged.resize((size_t) ci * co * sizeof(float));
            float * w = (float *) staged.data();
            for (int o = 0; o < co; ++o)
                for (int c = 0; c < ci; ++c) w[(size_t) c * co + o] = host[(size_t) o * ci + c];
            break;
        }
        case kLayoutVector: {
            staged.resize(count * sizeof(float));
            memcpy(staged.data(), host, count * sizeof(float));
            break;
        }
        default:
            return fail(be, TRELLIS_STATUS_ERROR, "unknown weight layout");
    }
    DevMem m;
    const trellis_status st = upload_bytes(be, staged.data(), staged.size(), &m);
    if (st != TRELLIS_STATUS_OK) return st;
    if (be->policy.cache_weights) {
        be->weights[key] = m;
    } else {
        be->transient.push_back(m);
    }
    *dev_out = m.ptr;
    return TRELLIS_STATUS_OK;
}

void end_call(Backend * be) {
    for (DevMem & m : be->transient) dev_release(be, &m);
    be->transient.clear();
}

struct CallScope {
    Backend * be;
    explicit CallScope(Backend * b) : be(b) { select_device(b); }
    ~CallScope() { end_call(be); }
};

// ---- ops ---------------------------------------------------------------------
void op_destroy(trellis_sparse_backend * backend);

trellis_status op_alloc_f32(trellis_sparse_backend * backend, size_t count, trellis_sparse_buffer ** out) {
    if (backend == nullptr || out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    Backend * be = as_backend(backend);
    CallScope scope(be);
    return new_buffer(be, count, be->policy.compute_dtype, out);
}

trellis_status op_upload_f32(trellis_sparse_backend * backend, const float * src, size_t count,
                             trellis_sparse_buffer ** out) {
    if (backend == nullptr || out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    if (src == nullptr && count != 0) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    CallScope scope(be);
    const int dt = be->policy.compute_dtype;
    trellis_sparse_buffer * b = nullptr;
    trellis_status st = new_buffer(be, count, dt, &b);
    if (st != TRELLIS_STATUS_OK) return st;
    if (count != 0) {
        if (dt == kF32) {
            hipError_t err = hipMemcpyAsync(b->ptr, src, count * 4, hipMemcpyHostToDevice, be->stream);
            if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
            st = hip_status(be, err, "upload_f32");
        } else {
            DevMem tmp;
            st = upload_bytes(be, src, count * 4, &tmp);
            if (st == TRELLIS_STATUS_OK) {
                st = hip_status(be, launch_convert_from_f32(dt, (const float *) tmp.ptr, b->ptr, (int64_t) count, be->stream),
                                "convert_from_f32");
            }
            dev_release(be, &tmp);
        }
    }
    if (st != TRELLIS_STATUS_OK) {
        DevMem m{b->ptr, b->cap};
        dev_release(be, &m);
        free(b);
        return st;
    }
    *out = b;
    return TRELLIS_STATUS_OK;
}

trellis_status op_upload_i32(trellis_sparse_backend * backend, const int32_t * src, size_t count,
                             trellis_sparse_buffer ** out) {
    if (backend == nullptr || out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    if (src == nullptr && count != 0) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    CallScope scope(be);
    trellis_sparse_buffer * b = nullptr;
    trellis_status st = new_buffer(be, count, -1, &b);
    if (st != TRELLIS_STATUS_OK) return st;
    if (count != 0) {
        hipError_t err = hipMemcpyAsync(b->ptr, src, count * 4, hipMemcpyHostToDevice, be->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
        st = hip_status(be, err, "upload_i32");
        if (st != TRELLIS_STATUS_OK) {
            DevMem m{b->ptr, b->cap};
            dev_release(be, &m);
            free(b);
            return st;
        }
    }
    *out = b;
    return TRELLIS_STATUS_OK;
}

trellis_status op_download_f32(trellis_sparse_backend * backend, const trellis_sparse_buffer * src, float * dst,
                               size_t count) {
    if (backend == nullptr || src == nullptr || dst == nullptr || count > src->count) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    Backend * be = as_backend(backend);
    CallScope scope(be);
    if (count == 0) return TRELLIS_STATUS_OK;
    if (src->dtype == kF32 || src->dtype < 0) {
        TSH_TRY(be, hipMemcpyAsync(dst, src->ptr, count * 4, hipMemcpyDeviceToHost, be->stream));
        TSH_TRY(be, hipStreamSynchronize(be->stream));
        return TRELLIS_STATUS_OK;
    }
    DevMem tmp;
    trellis_status st = dev_alloc(be, count * 4, &tmp);
    if (st != TRELLIS_STATUS_OK) return st;
    hipError_t err = launch_convert_to_f32(src->dtype, src->ptr, (float *) tmp.ptr, (int64_t) count, be->stream);
    if (err == hipSuccess) err = hipMemcpyAsync(dst, tmp.ptr, count * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    dev_release(be, &tmp);
    return hip_status(be, err, "download_f32");
}

void op_free_buffer(trellis_sparse_backend * backend, trellis_sparse_buffer * buffer) {
    if (backend == nullptr || buffer == nullptr) return;
    Backend * be = as_backend(backend);
    DevMem m{buffer->ptr, buffer->cap};
    dev_release(be, &m);
    free(buffer);
}

// y = x W^T + b (then SiLU).  With a residual (no SiLU): y = residual +
// (x W^T + b), residual [n][co] (may be y): the GEMM library adds it to the
// fp32 sums before the one rounding; the kernels write the rounded linear
// output to scratch ([n][co], neither y nor residual) and the add kernel
// forms the sum.
trellis_status linear_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * weight,
                           const float * bias, trellis_sparse_buffer * y, int64_t n, int ci, int co, int silu,
                           const trellis_sparse_buffer * residual = nullptr, trellis_sparse_buffer * scratch = nullptr) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (weight == nullptr || n <= 0 || ci <= 0 || co <= 0 || !float_buffer_ok(be, x, (size_t) n * ci) ||
        !float_buffer_ok(be, y, (size_t) n * co) ||
        (residual != nullptr && (silu || !float_buffer_ok(be, residual, (size_t) n * co) ||
                                 !float_buffer_ok(be, scratch, (size_t) n * co) || scratch->ptr == y->ptr ||
                                 scratch->ptr == residual->ptr))) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "linear: bad argument");
    }
    CallScope scope(be);
    const void * wt = nullptr;
    const void * bd = nullptr;
    const int dt = be->policy.compute_dtype;
    // bf16/fp16 with Ci = 64 or Ci % 128 == 0 and Co % 64 == 0: MFMA kernel;
    // Co <= 16 (the subdivide logits): the narrow MFMA kernel; otherwise (and
    // always for fp32) the reference-order VALU kernel.
    trellis_status st = get_weight(be, bias, (size_t) co, kLayoutVector, 0, co, &bd);
    if (st != TRELLIS_STATUS_OK) return st;
    // Wide shapes: the platform GEMM library when it has a plan (workspace
    // from the pool on first use; without it, or without a plan, the kernels
    // below run).
    if (be->policy.linear_algo == TRELLIS_SPARSE_HIP_LINEAR_AUTO && linear_lt_wanted(dt, n, ci, co)) {
        constexpr size_t kLtWorkspace = size_t(32) << 20;
        if (be->lt == nullptr) be->lt = linear_lt_create();
        if (be->lt_ws.ptr == nullptr && dev_alloc(be, kLtWorkspace, &be->lt_ws) != TRELLIS_STATUS_OK) {
            be->last_error.clear();
        }
        const void * w16 = nullptr;
        if (be->lt_ws.ptr != nullptr) {
            st = get_weight(be, weight, (size_t) ci * co, kLayoutLinear16, ci, co, &w16);
            if (st != TRELLIS_STATUS_OK) return st;
            stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
            const bool done =
                linear_lt_run(be->lt, dt, x->ptr, w16, (const float *) bd, residual ? residual->ptr : nullptr, y->ptr,
                              n, ci, co, silu, be->lt_ws.ptr, be->lt_ws.bytes, be->stream);
            stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
            if (done) return TRELLIS_STATUS_OK;
        }
    }
    const bool mfma = linear_mfma_supported(dt, ci, co);
    const bool narrow = !mfma && linear_narrow_supported(dt, ci, co);
    const int layout = mfma ? kLayoutLinearMfma : (narrow ? kLayoutLinear16 : kLayoutLinearT);
    st = get_weight(be, weight, (size_t) ci * co, layout, ci, co, &wt);
    if (st != TRELLIS_STATUS_OK) return st;
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    hipError_t err;
    void * out = residual != nullptr ? scratch->ptr : y->ptr;
    if (mfma) {
        err = launch_linear_mfma(dt, x->ptr, wt, (const float *) bd, out, n, ci, co, silu, be->cus, be->stream);
    } else if (narrow) {
        err = launch_linear_narrow(dt, x->ptr, wt, (const float *) bd, out, n, ci, co, silu, be->cus, be->stream);
    } else {
        err = launch_linear(dt, x->ptr, (const float *) wt, (const float *) bd, out, n, ci, co, silu, be->stream);
    }
    if (err == hipSuccess && residual != nullptr) {
        err = launch_add(dt, residual->ptr, out, y->ptr, n * co, be->stream);
    }
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    return hip_status(be, err, "linear");
}

trellis_status op_linear(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * weight,
                         const float * bias, trellis_sparse_buffer * y, int64_t n, int ci, int co) {
    return linear_impl(backend, x, weight, bias, y, n, ci, co, 0);
}

trellis_status op_linear_silu(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * weight,
                              const float * bias, trellis_sparse_buffer * y, int64_t n, int ci, int co) {
    return linear_impl(backend, x, weight, bias, y, n, ci, co, 1);
}

trellis_status norm_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * gamma,
                         const float * beta, trellis_sparse_buffer * y, int64_t n, int c, float eps, int silu);

// The tail at c >= 512 (a multiple of 128), where a tile's normalised rows
// would fill the LDS: row_norm into an n x c intermediate, mlp0 + SiLU into
// an n x 4c intermediate, and mlp2 with the residual added to its fp32 sums
// (GEMM library epilogue; the kernels' fallback adds the rounded mlp2 output
// as the slot sequence does).  The n x c intermediate is mlp2's scratch for
// that fallback.
bool mlp_composed_supported(int dtype, int c) { return (dtype == kF16 || dtype == kBF16) && c >= 512 && c % 128 == 0; }

trellis_status mlp_composed(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * gamma,
                            const float * beta, const float * w0, const float * b0, const float * w2,
                            const float * b2, const trellis_sparse_buffer * residual, trellis_sparse_buffer * y,
                            int64_t n, int c, float eps) {
    trellis_sparse_buffer *xn = nullptr, *hid = nullptr;
    trellis_status st = op_alloc_f32(backend, (size_t) n * c, &xn);
    if (st == TRELLIS_STATUS_OK) st = op_alloc_f32(backend, (size_t) n * 4 * c, &hid);
    if (st == TRELLIS_STATUS_OK) st = norm_impl(backend, x, gamma, beta, xn, n, c, eps, 0);
    if (st == TRELLIS_STATUS_OK) st = linear_impl(backend, xn, w0, b0, hid, n, c, 4 * c, 1);
    if (st == TRELLIS_STATUS_OK) st = linear_impl(backend, hid, w2, b2, y, n, 4 * c, c, 0, residual, xn);
    if (hid != nullptr) op_free_buffer(backend, hid);
    if (xn != nullptr) op_free_buffer(backend, xn);
    return st;
}

// The ConvNeXt block's MLP tail: y = residual + W2 SiLU(W0 LN(x) + b0) + b2,
// in one kernel for c = 64, 128 and 256, composed for wider rows.
trellis_status mlp_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * gamma,
                        const float * beta, const float * w0, const float * b0, const float * w2, const float * b2,
                        const trellis_sparse_buffer * residual, trellis_sparse_buffer * y, int64_t n, int c,
                        float eps) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (w0 == nullptr || w2 == nullptr || n <= 0 || c <= 0 || !(eps >= 0.0f) ||
        !float_buffer_ok(be, x, (size_t) n * c) || !float_buffer_ok(be, residual, (size_t) n * c) ||
        !float_buffer_ok(be, y, (size_t) n * c)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "convnext_mlp: bad argument");
    }
    if (!convnext_mlp_supported(be->policy.compute_dtype, c)) {
        if (mlp_composed_supported(be->policy.compute_dtype, c)) {
            return mlp_composed(backend, x, gamma, beta, w0, b0, w2, b2, residual, y, n, c, eps);
        }
        return fail(be, TRELLIS_STATUS_NOT_IMPLEMENTED,
                    "convnext_mlp: needs bf16/fp16 storage and c = 64, 128, 256 or a multiple of 128 from 512");
    }
    CallScope scope(be);
    const void *g = nullptr, *bt = nullptr, *pw0 = nullptr, *pb0 = nullptr, *pw2 = nullptr, *pb2 = nullptr;
    trellis_status st = get_weight(be, gamma, (size_t) c, kLayoutVector, 0, c, &g);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, beta, (size_t) c, kLayoutVector, 0, c, &bt);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, w0, (size_t) c * 4 * c, kLayoutMlp0, c, 4 * c, &pw0);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, b0, (size_t) 4 * c, kLayoutVector, 0, 4 * c, &pb0);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, w2, (size_t) 4 * c * c, kLayoutMlp2, 4 * c, c, &pw2);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, b2, (size_t) c, kLayoutVector, 0, c, &pb2);
    if (st != TRELLIS_STATUS_OK) return st;
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    const hipError_t err =
        launch_convnext_mlp(be->policy.compute_dtype, x->ptr, (const float *) g, (const float *) bt, pw0,
                            (const float *) pb0, pw2, (const float *) pb2, residual->ptr, y->ptr, n, c, eps,
                            be->cus, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    return hip_status(be, err, "convnext_mlp");
}

trellis_status norm_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * gamma,
                         const float * beta, trellis_sparse_buffer * y, int64_t n, int c, float eps, int silu) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (n <= 0 || c <= 0 || !(eps > 0.0f) || !float_buffer_ok(be, x, (size_t) n * c) ||
        !float_buffer_ok(be, y, (size_t) n * c)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "row_norm: bad argument");
    }
    CallScope scope(be);
    const void * g = nullptr;
    const void * b = nullptr;
    trellis_status st = get_weight(be, gamma, (size_t) c, kLayoutVector, 0, c, &g);
    if (st == TRELLIS_STATUS_OK) st = get_weight(be, beta, (size_t) c, kLayoutVector, 0, c, &b);
    if (st != TRELLIS_STATUS_OK) return st;
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    const hipError_t err = launch_row_norm(be->policy.compute_dtype, x->ptr, (const float *) g, (const float *) b,
                                           y->ptr, n, c, eps, silu, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    return hip_status(be, err, "row_norm");
}

trellis_status op_row_norm(trellis_sparse_backend * backend, const trellis_sparse_buffer * x, const float * gamma,
                           const float * beta, trellis_sparse_buffer * y, int64_t n, int c, float eps) {
    return norm_impl(backend, x, gamma, beta, y, n, c, eps, 0);
}

trellis_status op_row_norm_silu(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                const float * gamma, const float * beta, trellis_sparse_buffer * y, int64_t n, int c,
                                float eps) {
    return norm_impl(backend, x, gamma, beta, y, n, c, eps, 1);
}

trellis_status op_silu_inplace(trellis_sparse_backend * backend, trellis_sparse_buffer * x, size_t count) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!float_buffer_ok(be, x, count)) return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "silu: bad argument");
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    const hipError_t err = launch_silu(be->policy.compute_dtype, x->ptr, (int64_t) count, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    return hip_status(be, err, "silu");
}

trellis_status op_add(trellis_sparse_backend * backend, const trellis_sparse_buffer * a,
                      const trellis_sparse_buffer * b, trellis_sparse_buffer * y, size_t count) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!float_buffer_ok(be, a, count) || !float_buffer_ok(be, b, count) || !float_buffer_ok(be, y, count)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "add: bad argument");
    }
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    const hipError_t err = launch_add(be->policy.compute_dtype, a->ptr, b->ptr, y->ptr, (int64_t) count, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
    return hip_status(be, err, "add");
}

// ---- rulebook -------------------------------------------------------------------
trellis_status map_pass(Backend * be, trellis_sparse_rulebook * r, hipStream_t s);

// The neighbour table of a rulebook built without it, written on first use.
trellis_status rulebook_ensure_nbr(Backend * be, const trellis_sparse_rulebook * rc) {
    auto * r = const_cast<trellis_sparse_rulebook *>(rc);
    if (r->nbr.ptr != nullptr) return TRELLIS_STATUS_OK;
    const trellis_status st = dev_alloc(be, (size_t) r->n * 27 * 4, &r->nbr);
    if (st != TRELLIS_STATUS_OK) return st;
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_MAP);
    const trellis_status mst = map_pass(be, r, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_MAP);
    return mst;
}
void rulebook_release(Backend * be, trellis_sparse_rulebook * r) {
    if (r == nullptr) return;
    DevMem * mems[] = {&r->coords_mem, &r->table, &r->pool, &r->counters, &r->nbr, &r->mask,
                       &r->tile_counts, &r->tile_off, &r->pair_src, &r->pair_dst};
    for (DevMem * m : mems) dev_release(be, m);
    delete r;
}

int64_t next_pow2(int64_t v) {
    int64_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Writes the neighbour table of a built map (a second pass of the map
// kernel, which rewrites the pair lists with the same values).
trellis_status map_pass(Backend * be, trellis_sparse_rulebook * r, hipStream_t s) {
    return hip_status(be,
                      launch_map_tiles(r->coords, r->n, (const uint64_t *) r->table.ptr,
                                       r->table_slots, (const int32_t *) r->pool.ptr, (int32_t *) r->nbr.ptr,
                                       (uint32_t *) r->mask.ptr, (int32_t *) r->tile_counts.ptr,
                                       (int32_t *) r->tile_off.ptr, (int32_t *) r->pair_src.ptr,
                                       (uint8_t *) r->pair_dst.ptr, (int32_t *) r->counters.ptr, s),
                      "kernel map");
}

// Builds the brick hash and the kernel map for device coordinates `coords`
// on stream s (the main stream unless given).  The [n][27] neighbour table
// is written only when want_nbr (fp32 backends, whose conv reads it, and the
// mesh extraction); the compacted conv reads the pair lists, and the
// consumers of the table build it on first use (rulebook_ensure_nbr).
trellis_status rulebook_build_device(Backend * be, const int32_t * coords, int64_t n, trellis_sparse_rulebook * r,
                                     hipStream_t s = nullptr, bool want_nbr = false) {
    if (s == nullptr) s = be->stream;
    want_nbr = want_nbr || be->policy.compute_dtype == kF32;
    r->n = n;
    r->coords = const_cast<int32_t *>(coords);
    r->table_slots = std::max<int64_t>(64, next_pow2(2 * n));
    r->n_tiles = (n + kMapTile - 1) / kMapTile;
    const size_t slots = (size_t) r->table_slots;
    struct Need {
        DevMem * m;
        size_t bytes;
    } need[] = {
        {&r->table, slots * 16},
        {&r->pool, (size_t) (pool_empty_brick(n) + 1) * kBrickCells * 4},
        {&r->counters, kCounterInts * 4},
        {&r->nbr, want_nbr ? (size_t) n * 27 * 4 : 0},
        {&r->mask, (size_t) n * 4},
        {&r->tile_counts, (size_t) r->n_tiles * 27 * 4},
        {&r->tile_off, (size_t) r->n_tiles * 27 * 4},
        {&r->pair_src, (size_t) r->n_tiles * kMapTile * 27 * 4},
        {&r->pair_dst, (size_t) r->n_tiles * kMapTile * 27},
    };
    for (const Need & q : need) {
        if (q.bytes == 0) continue;
        const trellis_status st = dev_alloc(be, q.bytes, q.m);
        if (st != TRELLIS_STATUS_OK) return st;
    }
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_HASH);
    TSH_TRY(be, launch_hash_clear((uint64_t *) r->table.ptr, r->table_slots, (int32_t *) r->counters.ptr,
                                  (int32_t *) r->pool.ptr, n, s));
    TSH_TRY(be, launch_brick_insert(coords, n, (uint64_t *) r->table.ptr, r->table_slots,
                                    (int32_t *) r->counters.ptr, (int32_t *) r->pool.ptr, s));
    TSH_TRY(be, launch_voxel_insert(coords, n, (const uint64_t *) r->table.ptr,
                                    r->table_slots, (int32_t *) r->pool.ptr, (int32_t *) r->counters.ptr, s));
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_HASH);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_MAP);
    // One pass: neighbours (when wanted), per-tile counts and list starts,
    // and each tile's pair lists in its fixed region.
    const trellis_status mst = map_pass(be, r, s);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_MAP);
    if (mst != TRELLIS_STATUS_OK) return mst;
    if (be->policy.reject_duplicates) {
        int32_t flags[4] = {0, 0, 0, 0};
        TSH_TRY(be, hipMemcpyAsync(flags, r->counters.ptr, sizeof(flags), hipMemcpyDeviceToHost, s));
        TSH_TRY(be, hipStreamSynchronize(s));
        if (flags[1] != 0) return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_rulebook: duplicate coordinates");
    }
    return TRELLIS_STATUS_OK;
}

// Pair positions (tile regions of kMapTile * 27 entries) fit int32.
bool n_ok(int64_t n) { return n > 0 && (n + kMapTile - 1) / kMapTile * kMapTile * 27 <= (int64_t) INT32_MAX; }

trellis_status op_build_rulebook(trellis_sparse_backend * backend, const int32_t * coords_bxyz, int64_t n,
                                 trellis_sparse_rulebook ** out) {
    if (backend == nullptr || coords_bxyz == nullptr || out == nullptr || n <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *out = nullptr;
    Backend * be = as_backend(backend);
    if (!n_ok(n)) return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_rulebook: n*27 must fit int32");
    CallScope scope(be);
    auto * r = new (std::nothrow) trellis_sparse_rulebook();
    if (r == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    trellis_status st = upload_bytes(be, coords_bxyz, (size_t) n * 16, &r->coords_mem);
    if (st == TRELLIS_STATUS_OK) st = rulebook_build_device(be, (const int32_t *) r->coords_mem.ptr, n, r);
    if (st != TRELLIS_STATUS_OK) {
        rulebook_release(be, r);
        return st;
    }
    *out = r;
    return TRELLIS_STATUS_OK;
}

// The conv, optionally with a fused epilogue (fused_epi != nullptr: row
// norm (+ SiLU) or residual add, compacted schedule only).  epi's gamma and
// beta are host pointers here; they go through the weight cache.
trellis_status conv_impl(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                         const trellis_sparse_buffer * feats, const float * weight, const float * bias,
                         trellis_sparse_buffer * out, int64_t n, int ci, int co, const ConvEpilogue * fused_epi,
                         const char * what) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (rulebook == nullptr || weight == nullptr || n <= 0 || ci <= 0 || co <= 0 || n != rulebook->n ||
        !float_buffer_ok(be, feats, (size_t) n * ci) || !float_buffer_ok(be, out, (size_t) n * co) ||
        feats->ptr == out->ptr) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, (std::string(what) + ": bad argument").c_str());
    }
    const int dt = be->policy.compute_dtype;
    ConvEpilogue epi;
    if (fused_epi != nullptr) {
        const bool algo_ok = be->policy.conv_algo == TRELLIS_SPARSE_HIP_CONV_AUTO ||
                             be->policy.conv_algo == TRELLIS_SPARSE_HIP_CONV_COMPACT;
        const bool shape_ok = fused_epi->mode == kEpiNorm ? co == 128 : co % 128 == 0;
        if (!algo_ok || !conv_stream_supported(dt, ci, co) || !shape_ok) {
            const std::string msg = std::string(what) +
                                    ": needs the compacted conv (16-bit, Ci 64 or a multiple of 128) and " +
                                    (fused_epi->mode == kEpiNorm ? "Co == 128" : "Co a multiple of 128");
            return fail(be, TRELLIS_STATUS_NOT_IMPLEMENTED, msg.c_str());
        }
        epi = *fused_epi;
    }
    CallScope scope(be);
    int algo = be->policy.conv_algo;
    if (algo == TRELLIS_SPARSE_HIP_CONV_AUTO) {
        // The streamed compacted schedule multiplies valid pairs only; where it
        // does not apply (Ci not 64 or a multiple of 128) the masked one, then the VALU one.
        algo = TRELLIS_SPARSE_HIP_CONV_COMPACT;
    }
    if (algo == TRELLIS_SPARSE_HIP_CONV_COMPACT && !conv_stream_supported(dt, ci, co)) {
        algo = TRELLIS_SPARSE_HIP_CONV_MASKED;
    }
    if (algo == TRELLIS_SPARSE_HIP_CONV_MASKED && !conv_mfma_supported(dt, ci, co)) {
        algo = TRELLIS_SPARSE_HIP_CONV_GENERIC;
    }
    const void * bd = nullptr;
    trellis_status st = get_weight(be, bias, (size_t) co, kLayoutVector, 0, co, &bd);
    if (st != TRELLIS_STATUS_OK) return st;
    if (epi.mode == kEpiNorm) {
        const void * g = nullptr;
        const void * b = nullptr;
        st = get_weight(be, epi.gamma, (size_t) co, kLayoutVector, 0, co, &g);
        if (st == TRELLIS_STATUS_OK) st = get_weight(be, epi.beta, (size_t) co, kLayoutVector, 0, co, &b);
        if (st != TRELLIS_STATUS_OK) return st;
        epi.gamma = (const float *) g;
        epi.beta = (const float *) b;
    }
    const size_t wcount = (size_t) co * 27 * ci;
    hipError_t err;
    if (algo == TRELLIS_SPARSE_HIP_CONV_MASKED || algo == TRELLIS_SPARSE_HIP_CONV_COMPACT) {
        const void * w = nullptr;
        st = get_weight(be, weight, wcount,
                        algo == TRELLIS_SPARSE_HIP_CONV_COMPACT ? kLayoutConvMfmaGrouped : kLayoutConvMfma, ci, co,
                        &w);
        if (st != TRELLIS_STATUS_OK) return st;
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_CONV);
        if (algo == TRELLIS_SPARSE_HIP_CONV_COMPACT && epi.mode == kEpiNone && conv_os_supported(dt, ci, co, n)) {
            // Ci = Co = 64: the output-stationary kernel over the same lists.
            err = launch_conv_os(dt, feats->ptr, (const int32_t *) rulebook->pair_src.ptr,
                                 (const int32_t *) rulebook->tile_off.ptr, (const uint32_t *) rulebook->mask.ptr, w,
                                 (const float *) bd, out->ptr, n, ci, co, be->stream);
        } else if (algo == TRELLIS_SPARSE_HIP_CONV_COMPACT) {
            err = launch_conv_mfma_stream(dt, feats->ptr, (const int32_t *) rulebook->pair_src.ptr,
                                          (const uint8_t *) rulebook->pair_dst.ptr,
                                          (const int32_t *) rulebook->tile_off.ptr,
                                          (const int32_t *) rulebook->tile_counts.ptr,
                                          (const uint32_t *) rulebook->mask.ptr, w, (const float *) bd, out->ptr, n,
                                          ci, co, be->stream, epi,
                                          (const int32_t *) rulebook->counters.ptr + kLayoutStats);
        } else {
            st = rulebook_ensure_nbr(be, rulebook);
            if (st != TRELLIS_STATUS_OK) return st;
            err = launch_conv_mfma_masked(dt, feats->ptr, (const int32_t *) rulebook->nbr.ptr,
                                          (const uint32_t *) rulebook->mask.ptr, w, (const float *) bd, out->ptr, n,
                                          ci, co, be->stream);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_CONV);
    } else {
        const void * w = nullptr;
        st = get_weight(be, weight, wcount, kLayoutConvF32, ci, co, &w);
        if (st != TRELLIS_STATUS_OK) return st;
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_CONV);
        st = rulebook_ensure_nbr(be, rulebook);
        if (st != TRELLIS_STATUS_OK) return st;
        err = launch_conv_generic(dt, feats->ptr, (const int32_t *) rulebook->nbr.ptr, (const float *) w,
                                  (const float *) bd, out->ptr, n, ci, co, be->stream);
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_CONV);
    }
    return hip_status(be, err, what);
}

trellis_status op_sparse_conv3d(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                const trellis_sparse_buffer * feats, const float * weight, const float * bias,
                                trellis_sparse_buffer * out, int64_t n, int ci, int co) {
    return conv_impl(backend, rulebook, feats, weight, bias, out, n, ci, co, nullptr, "sparse_conv3d");
}

trellis_status conv_norm_impl(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                              const trellis_sparse_buffer * feats, const float * weight, const float * bias,
                              const float * gamma, const float * beta, float eps, int silu,
                              trellis_sparse_buffer * out, int64_t n, int ci, int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    if (!(eps > 0.0f)) return fail(as_backend(backend), TRELLIS_STATUS_INVALID_ARGUMENT, "conv_norm: bad argument");
    ConvEpilogue epi;
    epi.mode = kEpiNorm;
    epi.silu = silu != 0;
    epi.eps = eps;
    epi.gamma = gamma;
    epi.beta = beta;
    return conv_impl(backend, rulebook, feats, weight, bias, out, n, ci, co, &epi, "conv_norm");
}

trellis_status conv_add_impl(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                             const trellis_sparse_buffer * feats, const float * weight, const float * bias,
                             const trellis_sparse_buffer * residual, trellis_sparse_buffer * out, int64_t n, int ci,
                             int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (n <= 0 || co <= 0 || !float_buffer_ok(be, residual, (size_t) n * co)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "conv_add: bad argument");
    }
    ConvEpilogue epi;
    epi.mode = kEpiAdd;
    epi.residual = residual->ptr;
    return conv_impl(backend, rulebook, feats, weight, bias, out, n, ci, co, &epi, "conv_add");
}

// The whole ConvNeXt block: out = h + MLP(LN(conv(h))): the conv into one
// n x C intermediate, then the fused tail, whose LN overlaps its second GEMM
// (measured faster than the LN in the conv's epilogue, which runs after the
// block's last MFMAs).
trellis_status block_impl(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                          const trellis_sparse_buffer * h, const float * conv_w, const float * conv_b,
                          const float * gamma, const float * beta, const float * w0, const float * b0,
                          const float * w2, const float * b2, trellis_sparse_buffer * out, int64_t n, int c,
                          float eps) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (rulebook == nullptr || conv_w == nullptr || w0 == nullptr || w2 == nullptr || n <= 0 || c <= 0 ||
        n != rulebook->n || !(eps > 0.0f) || !float_buffer_ok(be, h, (size_t) n * c) ||
        !float_buffer_ok(be, out, (size_t) n * c) || h->ptr == out->ptr) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "convnext_block: bad argument");
    }
    const int dt = be->policy.compute_dtype;
    if (!convnext_mlp_supported(dt, c) && !mlp_composed_supported(dt, c)) {
        return fail(be, TRELLIS_STATUS_NOT_IMPLEMENTED,
                    "convnext_block: needs bf16/fp16 storage and c = 64, 128, 256 or a multiple of 128 from 512");
    }
    trellis_sparse_buffer * tmp = nullptr;
    trellis_status st = op_alloc_f32(backend, (size_t) n * c, &tmp);
    if (st != TRELLIS_STATUS_OK) return st;
    st = conv_impl(backend, rulebook, h, conv_w, conv_b, tmp, n, c, c, nullptr, "convnext_block");
    if (st == TRELLIS_STATUS_OK) st = mlp_impl(backend, tmp, gamma, beta, w0, b0, w2, b2, h, out, n, c, eps);
    op_free_buffer(backend, tmp);
    return st;
}

void op_free_rulebook(trellis_sparse_backend * backend, trellis_sparse_rulebook * rulebook) {
    if (backend == nullptr || rulebook == nullptr) return;
    rulebook_release(as_backend(backend), rulebook);
}

// ---- subdivide (C2S) --------------------------------------------------------------
trellis_status upload_index_pair(Backend * be, const int32_t * a, const int32_t * b, int64_t n, DevMem * da,
                                 DevMem * db) {
    trellis_status st = upload_bytes(be, a, (size_t) n * 4, da);
    if (st == TRELLIS_STATUS_OK) st = upload_bytes(be, b, (size_t) n * 4, db);
    return st;
}

trellis_status op_c2s_gather(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                             const int32_t * parent, const int32_t * subidx, trellis_sparse_buffer * y, int64_t n_out,
                             int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (x == nullptr || y == nullptr || parent == nullptr || subidx == nullptr || n_out <= 0 || co <= 0 ||
        !float_buffer_ok(be, y, (size_t) n_out * co) || x->dtype != be->policy.compute_dtype || x->ptr == nullptr) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "c2s_gather: bad argument");
    }
    CallScope scope(be);
    // Every parent index must address a row of x ([n_parent][8*co]).
    const int64_t x_rows = (int64_t) (x->count / ((size_t) co * 8));
    for (int64_t r = 0; r < n_out; ++r) {
        if (parent[r] < 0 || parent[r] >= x_rows || subidx[r] < 0 || subidx[r] > 7) {
            return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "c2s_gather: parent/subidx out of range");
        }
    }
    DevMem dp, ds;
    trellis_status st = upload_index_pair(be, parent, subidx, n_out, &dp, &ds);
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
        st = hip_status(be, launch_c2s_gather(be->policy.compute_dtype, x->ptr, (const int32_t *) dp.ptr,
                                              (const int32_t *) ds.ptr, y->ptr, n_out, co, be->stream),
                        "c2s_gather");
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    }
    dev_release(be, &dp);
    dev_release(be, &ds);
    return st;
}

trellis_status op_skip_repeat(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                              const int32_t * parent, const int32_t * subidx, trellis_sparse_buffer * y,
                              int64_t n_out, int ci, int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (x == nullptr || y == nullptr || parent == nullptr || subidx == nullptr || n_out <= 0 || ci <= 0 || co <= 0 ||
        !float_buffer_ok(be, y, (size_t) n_out * co) || x->dtype != be->policy.compute_dtype || x->ptr == nullptr) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "skip_repeat: bad argument");
    }
    CallScope scope(be);
    const int64_t x_rows = (int64_t) (x->count / (size_t) ci);
    for (int64_t r = 0; r < n_out; ++r) {
        if (parent[r] < 0 || parent[r] >= x_rows || subidx[r] < 0 || subidx[r] > 7) {
            return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "skip_repeat: parent/subidx out of range");
        }
    }
    DevMem dp, ds;
    trellis_status st = upload_index_pair(be, parent, subidx, n_out, &dp, &ds);
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
        st = hip_status(be, launch_skip_repeat(be->policy.compute_dtype, x->ptr, (const int32_t *) dp.ptr,
                                               (const int32_t *) ds.ptr, y->ptr, n_out, ci, co, be->stream),
                        "skip_repeat");
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    }
    dev_release(be, &dp);
    dev_release(be, &ds);
    return st;
}

void map_release(Backend * be, trellis_sparse_c2s_device_map * m) {
    if (m == nullptr) return;
    dev_release(be, &m->coords);
    dev_release(be, &m->parent);
    dev_release(be, &m->subidx);
    dev_release(be, &m->child);
    delete m;
}

bool map_known(const Backend * be, const trellis_sparse_c2s_device_map * m) {
    return m != nullptr && std::find(be->maps.begin(), be->maps.end(), m) != be->maps.end();
}

// Count -> exclusive scan -> fill, with the child total read back once.
trellis_status c2s_build(Backend * be, const int32_t * coords_dev, const trellis_sparse_buffer * logits, int64_t n,
                         trellis_sparse_c2s_device_map ** map_out) {
    *map_out = nullptr;
    DevMem counts, offsets, total, tmp;
    hipStream_t s = be->stream;
    trellis_status st = dev_alloc(be, (size_t) n * 4, &counts);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &offsets);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, 16, &total);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, scan_tmp_bytes(n), &tmp);
    int32_t m = 0;
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        hipError_t err = launch_c2s_count(be->policy.compute_dtype, logits->ptr, n, (int32_t *) counts.ptr, s);
        if (err == hipSuccess) {
            err = launch_scan_exclusive((const int32_t *) counts.ptr, (int32_t *) offsets.ptr, n,
                                        (int32_t *) total.ptr, tmp.ptr, s);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        if (err == hipSuccess) err = read_words(be, s, &m, total.ptr, 1);
        st = hip_status(be, err, "c2s count/scan");
    }
    if (st == TRELLIS_STATUS_OK && m <= 0) {
        st = fail(be, TRELLIS_STATUS_ERROR, "subdivide produced no children (all logits <= 0)");
    }
    trellis_sparse_c2s_device_map * map = nullptr;
    if (st == TRELLIS_STATUS_OK) {
        map = new (std::nothrow) trellis_sparse_c2s_device_map();
        if (map == nullptr) st = TRELLIS_STATUS_OUT_OF_MEMORY;
    }
    if (st == TRELLIS_STATUS_OK) {
        map->n = m;
        map->n_parent = n;
        st = dev_alloc(be, (size_t) m * 16, &map->coords);
        if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) m * 4, &map->parent);
        if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) m * 4, &map->subidx);
    }
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        st = hip_status(be,
                        launch_c2s_fill(be->policy.compute_dtype, coords_dev, logits->ptr,
                                        (const int32_t *) offsets.ptr, n, (int32_t *) map->coords.ptr,
                                        (int32_t *) map->parent.ptr, (int32_t *) map->subidx.ptr, s),
                        "c2s_fill");
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
    }
    dev_release(be, &counts);
    dev_release(be, &offsets);
    dev_release(be, &total);
    dev_release(be, &tmp);
    if (st != TRELLIS_STATUS_OK) {
        map_release(be, map);
        return st;
    }
    *map_out = map;
    return TRELLIS_STATUS_OK;
}

trellis_status op_build_c2s_map(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                const trellis_sparse_buffer * logits, int64_t n, int32_t ** coords_out,
                                int32_t ** parent_out, int32_t ** subidx_out, int64_t * n_out) {
    if (backend == nullptr || coords_bxyz == nullptr || coords_out == nullptr || parent_out == nullptr ||
        subidx_out == nullptr || n_out == nullptr || n <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *coords_out = nullptr;
    *parent_out = nullptr;
    *subidx_out = nullptr;
    *n_out = 0;
    Backend * be = as_backend(backend);
    if (!float_buffer_ok(be, logits, (size_t) n * 8) || n > INT32_MAX / 8) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_c2s_map: bad argument");
    }
    CallScope scope(be);
    DevMem cd;
    trellis_status st = upload_bytes(be, coords_bxyz, (size_t) n * 16, &cd);
    trellis_sparse_c2s_device_map * map = nullptr;
    if (st == TRELLIS_STATUS_OK) st = c2s_build(be, (const int32_t *) cd.ptr, logits, n, &map);
    dev_release(be, &cd);
    if (st != TRELLIS_STATUS_OK) return st;
    const int64_t m = map->n;
    int32_t * hc = (int32_t *) malloc((size_t) m * 16);
    int32_t * hp = (int32_t *) malloc((size_t) m * 4);
    int32_t * hs = (int32_t *) malloc((size_t) m * 4);
    if (hc == nullptr || hp == nullptr || hs == nullptr) {
        st = TRELLIS_STATUS_OUT_OF_MEMORY;
    } else {
        hipError_t err = hipMemcpyAsync(hc, map->coords.ptr, (size_t) m * 16, hipMemcpyDeviceToHost, be->stream);
        if (err == hipSuccess) err = hipMemcpyAsync(hp, map->parent.ptr, (size_t) m * 4, hipMemcpyDeviceToHost, be->stream);
        if (err == hipSuccess) err = hipMemcpyAsync(hs, map->subidx.ptr, (size_t) m * 4, hipMemcpyDeviceToHost, be->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
        st = hip_status(be, err, "build_c2s_map download");
    }
    map_release(be, map);
    if (st != TRELLIS_STATUS_OK) {
        free(hc);
        free(hp);
        free(hs);
        return st;
    }
    *coords_out = hc;
    *parent_out = hp;
    *subidx_out = hs;
    *n_out = m;
    return TRELLIS_STATUS_OK;
}

trellis_status op_alias_c2s_map(trellis_sparse_backend * backend, const int32_t * coords_bxyz, const int32_t * parent,
                                const int32_t * subidx, int64_t n, const int32_t * alias_coords_bxyz,
                                const int32_t * alias_parent, const int32_t * alias_subidx) {
    // A cache hint in the Vulkan backend (trellis_sparse_vulkan.c:2849-2878).
    // This backend keeps no host-pointer cache, so there is nothing to alias.
    if (backend == nullptr || coords_bxyz == nullptr || parent == nullptr || subidx == nullptr ||
        alias_coords_bxyz == nullptr || alias_parent == nullptr || alias_subidx == nullptr || n <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    return TRELLIS_STATUS_OK;
}

trellis_status op_build_c2s_map_device(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                       const trellis_sparse_c2s_device_map * coords_map,
                                       const trellis_sparse_buffer * logits, int64_t n,
                                       trellis_sparse_c2s_device_map ** map_out, int64_t * n_out) {
    if (backend == nullptr || map_out == nullptr || n_out == nullptr || (coords_bxyz == nullptr && coords_map == nullptr) ||
        n <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *map_out = nullptr;
    *n_out = 0;
    Backend * be = as_backend(backend);
    if (!float_buffer_ok(be, logits, (size_t) n * 8) || n > INT32_MAX / 8) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_c2s_map_device: bad argument");
    }
    if (coords_map != nullptr && (!map_known(be, coords_map) || coords_map->n != n)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_c2s_map_device: unknown coords_map or n mismatch");
    }
    CallScope scope(be);
    DevMem cd;
    const int32_t * coords_dev = nullptr;
    trellis_status st = TRELLIS_STATUS_OK;
    if (coords_map != nullptr) {
        coords_dev = (const int32_t *) coords_map->coords.ptr;
    } else {
        st = upload_bytes(be, coords_bxyz, (size_t) n * 16, &cd);
        coords_dev = (const int32_t *) cd.ptr;
    }
    trellis_sparse_c2s_device_map * map = nullptr;
    if (st == TRELLIS_STATUS_OK) st = c2s_build(be, coords_dev, logits, n, &map);
    dev_release(be, &cd);
    if (st != TRELLIS_STATUS_OK) return st;
    be->maps.push_back(map);
    *map_out = map;
    *n_out = map->n;
    return TRELLIS_STATUS_OK;
}

trellis_status op_build_rulebook_for_c2s_map(trellis_sparse_backend * backend,
                                             const trellis_sparse_c2s_device_map * map, trellis_sparse_rulebook ** out) {
    if (backend == nullptr || out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    Backend * be = as_backend(backend);
    if (!map_known(be, map)) return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_rulebook_for_c2s_map: unknown map");
    if (!n_ok(map->n)) return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_rulebook_for_c2s_map: n too large");
    CallScope scope(be);
    auto * r = new (std::nothrow) trellis_sparse_rulebook();
    if (r == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    // Built on the backend stream, in call order: a second stream that let
    // the build overlap the caller's next work (the feature broadcast of
    // config 3) made that phase longer, as the two kernels share the CUs and
    // HBM (config-3 step 2.061 -> 2.023 ms without it).  The map owns the
    // coordinates and outlives the rulebook.
    const trellis_status st = rulebook_build_device(be, (const int32_t *) map->coords.ptr, map->n, r);
    if (st != TRELLIS_STATUS_OK) {
        rulebook_release(be, r);
        return st;
    }
    *out = r;
    return TRELLIS_STATUS_OK;
}

trellis_status op_c2s_gather_device(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                    const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y,
                                    int64_t n_out, int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || map->parent.ptr == nullptr || x == nullptr || x->dtype != be->policy.compute_dtype ||
        x->ptr == nullptr || n_out != map->n || co <= 0 || !float_buffer_ok(be, y, (size_t) n_out * co) ||
        x->count < (size_t) map->n_parent * 8u * (size_t) co) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "c2s_gather_device: bad argument");
    }
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    const hipError_t err = launch_c2s_gather(be->policy.compute_dtype, x->ptr, (const int32_t *) map->parent.ptr,
                                             (const int32_t *) map->subidx.ptr, y->ptr, n_out, co, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    return hip_status(be, err, "c2s_gather_device");
}

trellis_status op_skip_repeat_device(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                     const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y,
                                     int64_t n_out, int ci, int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || map->parent.ptr == nullptr || x == nullptr || x->dtype != be->policy.compute_dtype ||
        x->ptr == nullptr || n_out != map->n || ci <= 0 || co <= 0 || !float_buffer_ok(be, y, (size_t) n_out * co) ||
        x->count < (size_t) map->n_parent * (size_t) ci) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "skip_repeat_device: bad argument");
    }
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    const hipError_t err = launch_skip_repeat(be->policy.compute_dtype, x->ptr, (const int32_t *) map->parent.ptr,
                                              (const int32_t *) map->subidx.ptr, y->ptr, n_out, ci, co, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    return hip_status(be, err, "skip_repeat_device");
}

trellis_status op_download_c2s_coords(trellis_sparse_backend * backend, const trellis_sparse_c2s_device_map * map,
                                      int32_t * coords_out, int64_t n) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || coords_out == nullptr || n != map->n) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "download_c2s_coords: bad argument");
    }
    CallScope scope(be);
    TSH_TRY(be, hipMemcpyAsync(coords_out, map->coords.ptr, (size_t) n * 16, hipMemcpyDeviceToHost, be->stream));
    TSH_TRY(be, hipStreamSynchronize(be->stream));
    return TRELLIS_STATUS_OK;
}

trellis_status op_download_c2s_map(trellis_sparse_backend * backend, const trellis_sparse_c2s_device_map * map,
                                   int32_t * coords_out, int32_t * parent_out, int32_t * subidx_out, int64_t n) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || map->parent.ptr == nullptr || coords_out == nullptr || parent_out == nullptr ||
        subidx_out == nullptr || n != map->n) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "download_c2s_map: bad argument");
    }
    CallScope scope(be);
    TSH_TRY(be, hipMemcpyAsync(coords_out, map->coords.ptr, (size_t) n * 16, hipMemcpyDeviceToHost, be->stream));
    TSH_TRY(be, hipMemcpyAsync(parent_out, map->parent.ptr, (size_t) n * 4, hipMemcpyDeviceToHost, be->stream));
    TSH_TRY(be, hipMemcpyAsync(subidx_out, map->subidx.ptr, (size_t) n * 4, hipMemcpyDeviceToHost, be->stream));
    TSH_TRY(be, hipStreamSynchronize(be->stream));
    return TRELLIS_STATUS_OK;
}

// ---- S2C downsample (encoder) -------------------------------------------------
// Radix sort of the coarse keys, heads, scan, emit; two small reads back (the
// field maxima that size the key, then the coarse count and error flags).
trellis_status s2c_build(Backend * be, const int32_t * fine_coords_host, const int32_t * fine_coords_dev, int64_t n,
                         trellis_sparse_c2s_device_map ** fine_out, trellis_sparse_c2s_device_map ** coarse_out) {
    hipStream_t s = be->stream;
    auto * fine = new (std::nothrow) trellis_sparse_c2s_device_map();
    auto * coarse = new (std::nothrow) trellis_sparse_c2s_device_map();
    if (fine == nullptr || coarse == nullptr) {
        delete fine;
        delete coarse;
        return TRELLIS_STATUS_OUT_OF_MEMORY;
    }
    fine->n = n;
    DevMem flags, part, klo[2], khi[2], row[2], hist, offs, total, tmp, head, excl;
    int32_t hf[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    trellis_status st = dev_alloc(be, (size_t) n * 16, &fine->coords);
    if (st == TRELLIS_STATUS_OK) {
        const hipMemcpyKind kind = fine_coords_host != nullptr ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
        const void * src = fine_coords_host != nullptr ? (const void *) fine_coords_host : (const void *) fine_coords_dev;
        st = hip_status(be, hipMemcpyAsync(fine->coords.ptr, src, (size_t) n * 16, kind, s), "s2c coords");
    }
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &fine->subidx);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, 32, &flags);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, s2c_prep_part_bytes(), &part);
    const int32_t * coords = (const int32_t *) fine->coords.ptr;
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        hipError_t err = launch_s2c_prep(coords, n, (int32_t *) fine->subidx.ptr, (int32_t *) part.ptr,
                                         (int32_t *) flags.ptr, s);
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        if (err == hipSuccess) err = hipMemcpyAsync(hf, flags.ptr, 32, hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);
        st = hip_status(be, err, "s2c prep");
    }
    if (st == TRELLIS_STATUS_OK && (hf[0] & 1)) {
        st = fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "s2c: negative coordinate");
    }
    int shifts[4] = {0, 0, 0, 0};
    const int key_bits = s2c_key_shape(hf + 1, shifts);
    const bool wide = key_bits > 64;
    const int64_t tiles = s2c_sort_tiles(n);
    for (int b = 0; b < 2 && st == TRELLIS_STATUS_OK; ++b) {
        st = dev_alloc(be, (size_t) n * 8, &klo[b]);
        if (st == TRELLIS_STATUS_OK && wide) st = dev_alloc(be, (size_t) n * 8, &khi[b]);
        if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &row[b]);
    }
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) tiles * 256 * 4, &hist);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) tiles * 256 * 4, &offs);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, 16, &total);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, s2c_sort_tmp_bytes(n), &tmp);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &head);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &excl);
    int cur = 0;
    int32_t m = 0;
    if (st == TRELLIS_STATUS_OK) {
        uint64_t * plo[2] = {(uint64_t *) klo[0].ptr, (uint64_t *) klo[1].ptr};
        uint64_t * phi[2] = {(uint64_t *) khi[0].ptr, (uint64_t *) khi[1].ptr};
        int32_t * prow[2] = {(int32_t *) row[0].ptr, (int32_t *) row[1].ptr};
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        hipError_t err = launch_s2c_sort(coords, n, shifts, key_bits, plo, phi, prow, (int32_t *) hist.ptr,
                                         (int32_t *) offs.ptr, (int32_t *) total.ptr, tmp.ptr, &cur, s);
        if (err == hipSuccess) {
            err = launch_s2c_heads(plo[cur], wide ? phi[cur] : nullptr, n, (int32_t *) head.ptr,
                                   (int32_t *) flags.ptr, s);
        }
        if (err == hipSuccess) {
            err = launch_scan_exclusive((const int32_t *) head.ptr, (int32_t *) excl.ptr, n, (int32_t *) total.ptr,
                                        tmp.ptr, s);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        if (err == hipSuccess) err = read_words(be, s, hf, flags.ptr, 1, &m, total.ptr, 1);
        st = hip_status(be, err, "s2c sort");
    }
    if (st == TRELLIS_STATUS_OK && (hf[0] & 2)) {
        st = fail(be, TRELLIS_STATUS_PARSE_ERROR, "s2c: the same fine voxel appears twice");
    }
    if (st == TRELLIS_STATUS_OK) {
        fine->n_parent = m;
        coarse->n = m;
        st = dev_alloc(be, (size_t) n * 4, &fine->parent);
        if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) m * 32, &fine->child);
        if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) m * 16, &coarse->coords);
    }
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        hipError_t err = launch_fill_i32((int32_t *) fine->child.ptr, (int64_t) m * 8, -1, s);
        if (err == hipSuccess) {
            err = launch_s2c_emit(coords, (const int32_t *) row[cur].ptr, (const int32_t *) fine->subidx.ptr,
                                  (const int32_t *) head.ptr, (const int32_t *) excl.ptr, n,
                                  (int32_t *) fine->parent.ptr, (int32_t *) coarse->coords.ptr,
                                  (int32_t *) fine->child.ptr, s);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE);
        st = hip_status(be, err, "s2c emit");
    }
    for (DevMem * d : {&flags, &part, &klo[0], &klo[1], &khi[0], &khi[1], &row[0], &row[1], &hist, &offs, &total, &tmp,
                       &head, &excl}) {
        dev_release(be, d);
    }
    if (st != TRELLIS_STATUS_OK) {
        map_release(be, fine);
        map_release(be, coarse);
        return st;
    }
    *fine_out = fine;
    *coarse_out = coarse;
    return TRELLIS_STATUS_OK;
}

trellis_status s2c_build_impl(trellis_sparse_backend * backend, const int32_t * fine_coords_bxyz,
                              const trellis_sparse_c2s_device_map * fine_coords_map, int64_t fine_n,
                              trellis_sparse_c2s_device_map ** fine_map_out,
                              trellis_sparse_c2s_device_map ** coarse_map_out, int64_t * coarse_n_out) {
    if (backend == nullptr || fine_map_out == nullptr || coarse_map_out == nullptr || coarse_n_out == nullptr ||
        (fine_coords_bxyz == nullptr && fine_coords_map == nullptr) || fine_n <= 0 || fine_n > INT32_MAX) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *fine_map_out = nullptr;
    *coarse_map_out = nullptr;
    *coarse_n_out = 0;
    Backend * be = as_backend(backend);
    if (fine_coords_map != nullptr && (!map_known(be, fine_coords_map) || fine_coords_map->n != fine_n)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "s2c_build_device: unknown fine_coords_map or n mismatch");
    }
    CallScope scope(be);
    trellis_sparse_c2s_device_map *fine = nullptr, *coarse = nullptr;
    const trellis_status st =
        s2c_build(be, fine_coords_map != nullptr ? nullptr : fine_coords_bxyz,
                  fine_coords_map != nullptr ? (const int32_t *) fine_coords_map->coords.ptr : nullptr, fine_n, &fine,
                  &coarse);
    if (st != TRELLIS_STATUS_OK) return st;
    be->maps.push_back(fine);
    be->maps.push_back(coarse);
    *fine_map_out = fine;
    *coarse_map_out = coarse;
    *coarse_n_out = coarse->n;
    return TRELLIS_STATUS_OK;
}

trellis_status s2c_pack_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                             const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y, int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || map->child.ptr == nullptr || co <= 0 || co % 8 != 0 ||
        !float_buffer_ok(be, x, (size_t) map->n * (size_t) (co / 8)) ||
        !float_buffer_ok(be, y, (size_t) map->n_parent * (size_t) co)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "s2c_pack_device: bad argument");
    }
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    const hipError_t err = launch_s2c_pack(be->policy.compute_dtype, x->ptr, (const int32_t *) map->child.ptr, y->ptr,
                                           map->n_parent, co, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    return hip_status(be, err, "s2c_pack_device");
}

trellis_status s2c_skip_mean_impl(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                  const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y, int ci,
                                  int co) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = as_backend(backend);
    if (!map_known(be, map) || map->child.ptr == nullptr || ci <= 0 || co <= 0 || co % 8 != 0 ||
        (8 * (int64_t) ci) % co != 0 || !float_buffer_ok(be, x, (size_t) map->n * (size_t) ci) ||
        !float_buffer_ok(be, y, (size_t) map->n_parent * (size_t) co)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "s2c_skip_mean_device: bad argument");
    }
    CallScope scope(be);
    stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    const hipError_t err = launch_s2c_skip_mean(be->policy.compute_dtype, x->ptr, (const int32_t *) map->child.ptr,
                                                y->ptr, map->n_parent, ci, co, be->stream);
    stage_end(be, TRELLIS_SPARSE_HIP_STAGE_BROADCAST);
    return hip_status(be, err, "s2c_skip_mean_device");
}

// ---- FlexiDualGrid mesh from decoder logits ------------------------------------
trellis_status fdg_mesh_impl(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                             const trellis_sparse_c2s_device_map * coords_map, const trellis_sparse_buffer * feats,
                             int64_t n, int channels, int resolution, trellis_mesh_host * mesh_out) {
    if (backend == nullptr || mesh_out == nullptr || (coords_bxyz == nullptr && coords_map == nullptr) || n < 0 ||
        n > INT32_MAX || channels < 7 || resolution <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    memset(mesh_out, 0, sizeof(*mesh_out));
    if (n == 0) return TRELLIS_STATUS_OK;
    Backend * be = as_backend(backend);
    if (!float_buffer_ok(be, feats, (size_t) n * (size_t) channels) || !n_ok(n) ||
        (coords_map != nullptr && (!map_known(be, coords_map) || coords_map->n != n))) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "flex_dual_grid_mesh: bad argument");
    }
    if (resolution > 65535) {
        // Corner lookups go through the kernel map, whose keys hold 16 bits per axis.
        return fail(be, TRELLIS_STATUS_NOT_IMPLEMENTED, "flex_dual_grid_mesh: resolution above 65535");
    }
    CallScope scope(be);
    hipStream_t s = be->stream;
    const int dt = be->policy.compute_dtype;
    DevMem cd, flags, vert, wgt, counts, first, total, tmp, faces;
    trellis_status st = TRELLIS_STATUS_OK;
    const int32_t * coords = nullptr;
    if (coords_map != nullptr) {
        coords = (const int32_t *) coords_map->coords.ptr;
    } else {
        st = upload_bytes(be, coords_bxyz, (size_t) n * 16, &cd);
        coords = (const int32_t *) cd.ptr;
    }
    auto * r = new (std::nothrow) trellis_sparse_rulebook();
    if (r == nullptr) st = TRELLIS_STATUS_OUT_OF_MEMORY;
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, 16, &flags);
    int32_t hf[4] = {0, 0, 0, 0}, dup[2] = {0, 0};
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
        hipError_t err = launch_fill_i32((int32_t *) flags.ptr, 4, 0, s);
        if (err == hipSuccess) {
            err = launch_fdg_check(dt, coords, feats->ptr, n, channels, resolution, (int32_t *) flags.ptr, s);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
        st = hip_status(be, err, "flex_dual_grid_mesh check");
    }
    if (st == TRELLIS_STATUS_OK) st = rulebook_build_device(be, coords, n, r, nullptr, true);
    if (st == TRELLIS_STATUS_OK) {
        hipError_t err = hipMemcpyAsync(hf, flags.ptr, 16, hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipMemcpyAsync(dup, r->counters.ptr, 8, hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);
        st = hip_status(be, err, "flex_dual_grid_mesh flags");
    }
    if (st == TRELLIS_STATUS_OK && hf[0] != 0) {
        st = fail(be, TRELLIS_STATUS_PARSE_ERROR,
                  "flex_dual_grid_mesh: batch index not 0, coordinate outside [0, resolution) or non-finite logit");
    }
    if (st == TRELLIS_STATUS_OK && dup[1] != 0) {
        st = fail(be, TRELLIS_STATUS_PARSE_ERROR, "flex_dual_grid_mesh: repeated coordinate");
    }
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 12, &vert);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &wgt);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &counts);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, (size_t) n * 4, &first);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, 16, &total);
    if (st == TRELLIS_STATUS_OK) st = dev_alloc(be, scan_tmp_bytes(n), &tmp);
    int32_t quads = 0;
    if (st == TRELLIS_STATUS_OK) {
        stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
        const int32_t * nbr = (const int32_t *) r->nbr.ptr;
        hipError_t err = launch_fdg_vertices(dt, coords, feats->ptr, n, channels, resolution, (float *) vert.ptr,
                                             (float *) wgt.ptr, s);
        if (err == hipSuccess) err = launch_fdg_count(dt, feats->ptr, nbr, n, channels, (int32_t *) counts.ptr, s);
        if (err == hipSuccess) {
            err = launch_scan_exclusive((const int32_t *) counts.ptr, (int32_t *) first.ptr, n, (int32_t *) total.ptr,
                                        tmp.ptr, s);
        }
        stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
        if (err == hipSuccess) err = read_words(be, s, &quads, total.ptr, 1);
        st = hip_status(be, err, "flex_dual_grid_mesh count");
    }
    if (st == TRELLIS_STATUS_OK && quads > 0) {
        st = dev_alloc(be, (size_t) quads * 24, &faces);
        if (st == TRELLIS_STATUS_OK) {
            stage_begin(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
            st = hip_status(be,
                            launch_fdg_faces(dt, feats->ptr, (const int32_t *) r->nbr.ptr, (const float *) wgt.ptr,
                                             (const int32_t *) first.ptr, n, channels, (int32_t *) faces.ptr, s),
                            "flex_dual_grid_mesh faces");
            stage_end(be, TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE);
        }
    }
    float * hv = nullptr;
    int32_t * hfaces = nullptr;
    if (st == TRELLIS_STATUS_OK) {
        hv = (float *) malloc((size_t) n * 12);
        hfaces = quads > 0 ? (int32_t *) malloc((size_t) quads * 24) : nullptr;
        if (hv == nullptr || (quads > 0 && hfaces == nullptr)) {
            st = TRELLIS_STATUS_OUT_OF_MEMORY;
        } else {
            // Both arrays through the pinned staging buffer (full-rate
            // transfers), then copied into the caller's malloc-owned arrays.
            const size_t vbytes = (size_t) n * 12, voff = (vbytes + 255) / 256 * 256;
            const size_t fbytes = (size_t) quads * 24;
            st = pinned_reserve(be, voff + fbytes);
            if (st == TRELLIS_STATUS_OK) {
                char * stage = (char *) be->pinned;
                hipError_t err = hipMemcpyAsync(stage, vert.ptr, vbytes, hipMemcpyDeviceToHost, s);
                if (err == hipSuccess && quads > 0) {
                    err = hipMemcpyAsync(stage + voff, faces.ptr, fbytes, hipMemcpyDeviceToHost, s);
                }
                if (err == hipSuccess) err = hipStreamSynchronize(s);
                st = hip_status(be, err, "flex_dual_grid_mesh download");
                if (st == TRELLIS_STATUS_OK) {
                    parallel_copy(hv, stage, vbytes);
                    if (quads > 0) parallel_copy(hfaces, stage + voff, fbytes);
                }
            }
        }
    }
    for (DevMem * d : {&cd, &flags, &vert, &wgt, &counts, &first, &total, &tmp, &faces}) dev_release(be, d);
    if (r != nullptr) rulebook_release(be, r);
    if (st != TRELLIS_STATUS_OK) {
        free(hv);
        free(hfaces);
        return st;
    }
    mesh_out->vertices = hv;
    mesh_out->vertex_colors = nullptr;
    mesh_out->faces = hfaces;
    mesh_out->n_vertices = n;
    mesh_out->n_faces = (int64_t) quads * 2;
    return TRELLIS_STATUS_OK;
}

trellis_status op_trim(trellis_sparse_backend * backend, unsigned flags, size_t * released_bytes) {
    if (released_bytes != nullptr) *released_bytes = 0;
    if (backend == nullptr || (flags & ~(unsigned) TRELLIS_SPARSE_TRIM_ALL) != 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    if (flags == 0) return TRELLIS_STATUS_OK;
    Backend * be = as_backend(backend);
    CallScope scope(be);
    TSH_TRY(be, hipStreamSynchronize(be->stream));
    size_t released = 0;
    if (flags & TRELLIS_SPARSE_TRIM_WEIGHTS) {
        for (auto & kv : be->weights) {
            released += kv.second.bytes;
            (void) hipFree(kv.second.ptr);
        }
        be->weights.clear();
    }
    if (flags & TRELLIS_SPARSE_TRIM_FREE_BUFFERS) {
        dev_release(be, &be->lt_ws);  // the GEMM library's workspace (taken again on the next wide linear)
        for (auto & kv : be->free_blocks) {
            for (void * p : kv.second) {
                (void) hipFree(p);
                released += kv.first;
            }
        }
        be->free_blocks.clear();
        if (be->pinned != nullptr) {
            (void) hipHostFree(be->pinned);
            released += be->pinned_bytes;
            be->pinned = nullptr;
            be->pinned_bytes = 0;
        }
        be->pooled_bytes = 0;
    }
    if (released_bytes != nullptr) *released_bytes = released;
    return TRELLIS_STATUS_OK;
}

trellis_status op_naf(trellis_sparse_backend *, const float *, const float *, const float *, const int32_t *, int64_t,
                      const struct trellis_pixal_camera *, const struct trellis_pixal_naf_attention_desc *, float *,
                      size_t) {
    // Pixal3D NAF attention is not part of the sparse-convolution path.
    return TRELLIS_STATUS_NOT_IMPLEMENTED;
}

const trellis_sparse_backend_ops g_ops = {
    op_destroy,
    op_alloc_f32,
    op_upload_f32,
    op_upload_i32,
    op_download_f32,
    op_free_buffer,
    op_linear,
    op_linear_silu,
    op_row_norm,
    op_row_norm_silu,
    op_silu_inplace,
    op_add,
    op_build_rulebook,
    op_sparse_conv3d,
    op_free_rulebook,
    op_c2s_gather,
    op_skip_repeat,
    op_build_c2s_map,
    op_alias_c2s_map,
    op_build_c2s_map_device,
    op_build_rulebook_for_c2s_map,
    op_c2s_gather_device,
    op_skip_repeat_device,
    op_download_c2s_coords,
    op_download_c2s_map,
    op_trim,
    op_naf,
};

void op_destroy(trellis_sparse_backend * backend) {
    if (backend == nullptr) return;
    Backend * be = as_backend(backend);
    select_device(be);
    (void) hipStreamSynchronize(be->stream);
    for (auto * m : be->maps) map_release(be, m);
    be->maps.clear();
    for (auto & kv : be->weights) dev_release(be, &kv.second);
    be->weights.clear();
    dev_release(be, &be->lt_ws);
    linear_lt_destroy(be->lt);
    be->lt = nullptr;
    for (auto & kv : be->free_blocks)
        for (void * p : kv.second) (void) hipFree(p);
    for (auto & m : be->pending) {
        (void) hipEventDestroy(m.a);
        (void) hipEventDestroy(m.b);
    }
    for (hipEvent_t e : be->spare_events) (void) hipEventDestroy(e);
    for (hipEvent_t e : be->user_events)
        if (e != nullptr) (void) hipEventDestroy(e);
    if (be->pinned != nullptr) (void) hipHostFree(be->pinned);
    if (be->host_words != nullptr) (void) hipHostFree(be->host_words);
    if (be->words_ready != nullptr) (void) hipEventDestroy(be->words_ready);
    (void) hipStreamDestroy(be->stream);
    delete be;
}

}  // namespace
}  // namespace tsh

using tsh::Backend;

extern "C" {

void trellis_sparse_hip_policy_init(trellis_sparse_hip_policy * policy) {
    if (policy == nullptr) return;
    memset(policy, 0, sizeof(*policy));
    policy->struct_size = sizeof(*policy);
    policy->compute_dtype = TRELLIS_SPARSE_HIP_F32;
    policy->conv_algo = TRELLIS_SPARSE_HIP_CONV_AUTO;
    policy->cache_weights = 1;
    policy->reject_duplicates = 0;
    policy->linear_algo = TRELLIS_SPARSE_HIP_LINEAR_AUTO;
}

int trellis_sparse_hip_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) {
        (void) hipGetLastError();
        return 0;
    }
    return count;
}

trellis_status trellis_sparse_hip_backend_create_ex(int device, const trellis_sparse_hip_policy * policy,
                                                    trellis_sparse_backend ** out) {
    if (out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    trellis_sparse_hip_policy p;
    trellis_sparse_hip_policy_init(&p);
    if (policy != nullptr) {
        if (policy->struct_size != sizeof(trellis_sparse_hip_policy)) return TRELLIS_STATUS_INVALID_ARGUMENT;
        p = *policy;
    }
    if (p.compute_dtype < TRELLIS_SPARSE_HIP_F32 || p.compute_dtype > TRELLIS_SPARSE_HIP_BF16 ||
        p.conv_algo < TRELLIS_SPARSE_HIP_CONV_AUTO || p.conv_algo > TRELLIS_SPARSE_HIP_CONV_COMPACT ||
        p.linear_algo < TRELLIS_SPARSE_HIP_LINEAR_AUTO || p.linear_algo > TRELLIS_SPARSE_HIP_LINEAR_KERNEL) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    const int count = trellis_sparse_hip_device_count();
    if (device < 0 || device >= count) return TRELLIS_STATUS_CUDA_UNAVAILABLE;
    if (hipSetDevice(device) != hipSuccess) {
        (void) hipGetLastError();
        return TRELLIS_STATUS_CUDA_UNAVAILABLE;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) {
        (void) hipGetLastError();
        return TRELLIS_STATUS_CUDA_UNAVAILABLE;
    }
    auto * be = new (std::nothrow) Backend();
    if (be == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    be->cus = cus;
    if (hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking) != hipSuccess) {
        (void) hipGetLastError();
        delete be;
        return TRELLIS_STATUS_CUDA_UNAVAILABLE;
    }
    // Small reads fall back to pageable copies and a stream synchronisation
    // when either of these is missing.
    if (hipHostMalloc((void **) &be->host_words, tsh::kHostWords * 4, hipHostMallocDefault) != hipSuccess) {
        (void) hipGetLastError();
        be->host_words = nullptr;
    }
    if (hipEventCreateWithFlags(&be->words_ready, hipEventDisableTiming) != hipSuccess) {
        (void) hipGetLastError();
        be->words_ready = nullptr;
    }
    be->base.ops = &tsh::g_ops;
    be->base.kind = TRELLIS_SPARSE_BACKEND_HIP;
    be->base.device = device;
    be->device = device;
    be->policy = p;
    be->into = tsh::scratch_for(device);
    // TRELLIS_HIP_FAIL_ALLOC_AFTER=N[,K]: the device allocation attempts after
    // the first N fail (K of them, default all), for out-of-memory tests.
    if (const char * env = getenv("TRELLIS_HIP_FAIL_ALLOC_AFTER")) {
        char * end = nullptr;
        const long long after = strtoll(env, &end, 10);
        long long count = INT64_MAX;
        if (end != nullptr && *end == ',') count = strtoll(end + 1, nullptr, 10);
        if (end != env && after >= 0 && count > 0) {
            be->fail_after = after;
            be->fail_count = count;
        }
    }
    *out = &be->base;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_fail_alloc(trellis_sparse_backend * backend, int64_t after, int64_t count) {
    if (backend == nullptr || (after >= 0 && count <= 0)) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    be->fail_after = after < 0 ? -1 : after;
    be->fail_count = after < 0 ? 0 : count;
    be->alloc_attempts = 0;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_backend_create(int device, trellis_sparse_backend ** out) {
    return trellis_sparse_hip_backend_create_ex(device, nullptr, out);
}

const char * trellis_sparse_hip_last_error(const trellis_sparse_backend * backend) {
    if (backend == nullptr) return "";
    return tsh::as_backend(backend)->last_error.c_str();
}

trellis_status trellis_sparse_hip_synchronize(trellis_sparse_backend * backend) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    return tsh::hip_status(be, hipStreamSynchronize(be->stream), "synchronize");
}

trellis_status trellis_sparse_hip_rulebook_stats(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook, int64_t * n,
                                                 int64_t * pairs, int64_t * table_slots, int64_t * bricks) {
    if (backend == nullptr || rulebook == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    int32_t ctr[tsh::kCounterInts];
    std::vector<int32_t> cnt((size_t) rulebook->n_tiles * 27);
    hipError_t err = hipMemcpyAsync(ctr, rulebook->counters.ptr, sizeof(ctr), hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(cnt.data(), rulebook->tile_counts.ptr, cnt.size() * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    if (err != hipSuccess) return tsh::hip_status(be, err, "rulebook_stats");
    int64_t total = 0;
    for (const int32_t c : cnt) total += c;
    int64_t nb = 0;
    for (int g = 0; g < tsh::kBrickCounters; ++g) nb += ctr[tsh::kBrickCounter + g];
    if (n != nullptr) *n = rulebook->n;
    if (pairs != nullptr) *pairs = total;
    if (table_slots != nullptr) *table_slots = rulebook->table_slots;
    if (bricks != nullptr) *bricks = nb;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_download_neighbors(trellis_sparse_backend * backend,
                                                     const trellis_sparse_rulebook * rulebook, int32_t * nbr_out,
                                                     int64_t n) {
    if (backend == nullptr || rulebook == nullptr || nbr_out == nullptr || n != rulebook->n) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    const trellis_status st = tsh::rulebook_ensure_nbr(be, rulebook);
    if (st != TRELLIS_STATUS_OK) return st;
    hipError_t err = hipMemcpyAsync(nbr_out, rulebook->nbr.ptr, (size_t) n * 27 * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    return tsh::hip_status(be, err, "download_neighbors");
}

trellis_status trellis_sparse_hip_download_pairs(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook, int64_t * counts_out,
                                                 int32_t * src_out, int32_t * dst_out, int64_t capacity) {
    if (backend == nullptr || rulebook == nullptr || counts_out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    // Per-offset totals are the column sums of the per-(tile, offset) counts.
    const int64_t tiles = rulebook->n_tiles;
    std::vector<int32_t> off((size_t) tiles * 27), cnt((size_t) tiles * 27);
    hipError_t err =
        hipMemcpyAsync(cnt.data(), rulebook->tile_counts.ptr, cnt.size() * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    if (err != hipSuccess) return tsh::hip_status(be, err, "download_pairs");
    int64_t total = 0;
    for (int k = 0; k < 27; ++k) {
        int64_t c = 0;
        for (int64_t t = 0; t < tiles; ++t) c += cnt[(size_t) t * 27 + k];
        counts_out[k] = c;
        total += c;
    }
    if (src_out == nullptr && dst_out == nullptr) return TRELLIS_STATUS_OK;
    if (total > capacity) return tsh::fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "download_pairs: capacity too small");
    // The device lists are tile-major; reorder them to the canonical
    // offset-major order (destination ascending within an offset).
    const size_t span = (size_t) tiles * tsh::kMapTile * 27;  // every tile's region
    std::vector<int32_t> hs(span);
    std::vector<uint8_t> hd(span);
    err = hipMemcpyAsync(off.data(), rulebook->tile_off.ptr, off.size() * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess && total > 0)
        err = hipMemcpyAsync(hs.data(), rulebook->pair_src.ptr, span * 4, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess && total > 0)
        err = hipMemcpyAsync(hd.data(), rulebook->pair_dst.ptr, span, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    if (err != hipSuccess) return tsh::hip_status(be, err, "download_pairs");
    int64_t at = 0;
    for (int k = 0; k < 27; ++k) {
        for (int64_t t = 0; t < tiles; ++t) {
            const int64_t from = off[(size_t) t * 27 + k], c = cnt[(size_t) t * 27 + k];
            if (c <= 0) continue;
            if (src_out != nullptr) memcpy(src_out + at, hs.data() + from, (size_t) c * 4);
            if (dst_out != nullptr) {
                for (int64_t j = 0; j < c; ++j) dst_out[at + j] = (int32_t) (t * tsh::kMapTile + hd[(size_t) (from + j)]);
            }
            at += c;
        }
    }
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_upload_raw(trellis_sparse_backend * backend, const void * src, size_t count,
                                             trellis_sparse_buffer ** out) {
    if (backend == nullptr || out == nullptr || (src == nullptr && count != 0)) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *out = nullptr;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    trellis_sparse_buffer * b = nullptr;
    trellis_status st = tsh::new_buffer(be, count, be->policy.compute_dtype, &b);
    if (st != TRELLIS_STATUS_OK) return st;
    if (count != 0) {
        hipError_t err = hipMemcpyAsync(b->ptr, src, b->bytes, hipMemcpyHostToDevice, be->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
        st = tsh::hip_status(be, err, "upload_raw");
    }
    if (st != TRELLIS_STATUS_OK) {
        tsh::op_free_buffer(backend, b);
        return st;
    }
    *out = b;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_download_raw(trellis_sparse_backend * backend, const trellis_sparse_buffer * src,
                                               void * dst, size_t count) {
    if (backend == nullptr || src == nullptr || dst == nullptr || count > src->count) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    const size_t elem = src->dtype < 0 ? 4u : tsh::dtype_bytes(src->dtype);
    hipError_t err = hipMemcpyAsync(dst, src->ptr, count * elem, hipMemcpyDeviceToHost, be->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(be->stream);
    return tsh::hip_status(be, err, "download_raw");
}

trellis_status trellis_sparse_hip_upload_coords(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                                int64_t n, trellis_sparse_c2s_device_map ** map_out) {
    if (backend == nullptr || coords_bxyz == nullptr || map_out == nullptr || n <= 0) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *map_out = nullptr;
    Backend * be = tsh::as_backend(backend);
    if (!tsh::n_ok(n)) return tsh::fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "upload_coords: n too large");
    tsh::select_device(be);
    auto * map = new (std::nothrow) trellis_sparse_c2s_device_map();
    if (map == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    map->n = n;
    const trellis_status st = tsh::upload_bytes(be, coords_bxyz, (size_t) n * 16, &map->coords);
    if (st != TRELLIS_STATUS_OK) {
        tsh::map_release(be, map);
        return st;
    }
    be->maps.push_back(map);
    *map_out = map;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_free_c2s_map(trellis_sparse_backend * backend, trellis_sparse_c2s_device_map * map) {
    if (backend == nullptr || map == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    auto it = std::find(be->maps.begin(), be->maps.end(), map);
    if (it == be->maps.end()) return tsh::fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "free_c2s_map: unknown map");
    be->maps.erase(it);
    tsh::select_device(be);
    tsh::map_release(be, map);
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_build_c2s_map_into(trellis_sparse_backend * backend,
                                                     const trellis_sparse_buffer * coords,
                                                     const trellis_sparse_buffer * logits, int64_t n,
                                                     trellis_sparse_buffer * coords_out,
                                                     trellis_sparse_buffer * parent_out,
                                                     trellis_sparse_buffer * subidx_out, int64_t * n_out) {
    using namespace tsh;
    if (backend == nullptr || n_out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *n_out = 0;
    Backend * be = as_backend(backend);
    const bool int_bufs = coords != nullptr && coords_out != nullptr && parent_out != nullptr &&
                          subidx_out != nullptr && coords->dtype < 0 && coords_out->dtype < 0 &&
                          parent_out->dtype < 0 && subidx_out->dtype < 0;
    if (n <= 0 || !int_bufs || coords->count < (size_t) n * 4 || !float_buffer_ok(be, logits, (size_t) n * 8)) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_c2s_map_into: bad argument");
    }
    if (n > kIntoMaxParents) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT,
                    "build_c2s_map_into: more than 1048576 parents (the size of its fixed scratch)");
    }
    if (be->into == nullptr) {
        return fail(be, TRELLIS_STATUS_ERROR, "build_c2s_map_into: scratch address unavailable on this device");
    }
    select_device(be);
    hipStream_t s = be->stream;
    IntoScratch & sc = *be->into;
    // One call at a time per device; this call's kernels start after the
    // previous call's fill, whatever stream it ran on.
    std::lock_guard<std::mutex> lock(sc.mu);
    int32_t * counts = (int32_t *) (sc.addr + kIntoCounts);
    int32_t * offsets = (int32_t *) (sc.addr + kIntoOffsets);
    int32_t * total = (int32_t *) (sc.addr + kIntoTotal);
    void * sums = sc.addr + kIntoSums;
    static_assert(kIntoSums + (kIntoMaxParents / 2048 + 2) * 4 <= kIntoScratchBytes, "scan sums fit");
    // Every counts and offsets entry below n, the total and the tile sums
    // are written before they are read, so nothing needs clearing.
    hipError_t err = hipStreamWaitEvent(s, sc.done, 0);
    if (err == hipSuccess) err = launch_c2s_count(be->policy.compute_dtype, logits->ptr, n, counts, s);
    if (err == hipSuccess) err = launch_scan_exclusive(counts, offsets, n, total, sums, s);
    int32_t m = 0;
    if (err == hipSuccess) err = read_words(be, s, &m, total, 1);
    if (err != hipSuccess) return hip_status(be, err, "build_c2s_map_into: count/scan");
    if (m <= 0) return fail(be, TRELLIS_STATUS_ERROR, "subdivide produced no children (all logits <= 0)");
    *n_out = m;
    if (coords_out->count < (size_t) m * 4 || parent_out->count < (size_t) m || subidx_out->count < (size_t) m) {
        return fail(be, TRELLIS_STATUS_INVALID_ARGUMENT, "build_c2s_map_into: outputs hold fewer than n_out children");
    }
    // (The returns above follow read_words, which waited for count and scan.)
    err = launch_c2s_fill(be->policy.compute_dtype, (const int32_t *) coords->ptr, logits->ptr, offsets, n,
                          (int32_t *) coords_out->ptr, (int32_t *) parent_out->ptr, (int32_t *) subidx_out->ptr, s);
    if (err == hipSuccess) err = hipEventRecord(sc.done, s);
    return hip_status(be, err, "build_c2s_map_into: fill");
}

trellis_status trellis_sparse_hip_s2c_build_device(trellis_sparse_backend * backend, const int32_t * fine_coords_bxyz,
                                                   const trellis_sparse_c2s_device_map * fine_coords_map,
                                                   int64_t fine_n, trellis_sparse_c2s_device_map ** fine_map_out,
                                                   trellis_sparse_c2s_device_map ** coarse_map_out,
                                                   int64_t * coarse_n_out) {
    return tsh::s2c_build_impl(backend, fine_coords_bxyz, fine_coords_map, fine_n, fine_map_out, coarse_map_out,
                               coarse_n_out);
}

trellis_status trellis_sparse_hip_s2c_pack_device(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                                  const trellis_sparse_c2s_device_map * fine_map,
                                                  trellis_sparse_buffer * y, int co) {
    return tsh::s2c_pack_impl(backend, x, fine_map, y, co);
}

trellis_status trellis_sparse_hip_s2c_skip_mean_device(trellis_sparse_backend * backend,
                                                       const trellis_sparse_buffer * x,
                                                       const trellis_sparse_c2s_device_map * fine_map,
                                                       trellis_sparse_buffer * y, int ci, int co) {
    return tsh::s2c_skip_mean_impl(backend, x, fine_map, y, ci, co);
}

trellis_status trellis_sparse_hip_flex_dual_grid_mesh(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                                     const trellis_sparse_c2s_device_map * coords_map,
                                                     const trellis_sparse_buffer * feats, int64_t n, int channels,
                                                     int resolution, trellis_mesh_host * mesh_out) {
    return tsh::fdg_mesh_impl(backend, coords_bxyz, coords_map, feats, n, channels, resolution, mesh_out);
}

trellis_status trellis_sparse_hip_convnext_mlp(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                               const float * gamma, const float * beta, const float * mlp0_w,
                                               const float * mlp0_b, const float * mlp2_w, const float * mlp2_b,
                                               const trellis_sparse_buffer * residual, trellis_sparse_buffer * y,
                                               int64_t n, int c, float eps) {
    return tsh::mlp_impl(backend, x, gamma, beta, mlp0_w, mlp0_b, mlp2_w, mlp2_b, residual, y, n, c, eps);
}

trellis_status trellis_sparse_hip_convnext_block(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook,
                                                 const trellis_sparse_buffer * h, const float * conv_w,
                                                 const float * conv_b, const float * gamma, const float * beta,
                                                 const float * mlp0_w, const float * mlp0_b, const float * mlp2_w,
                                                 const float * mlp2_b, trellis_sparse_buffer * out, int64_t n, int c,
                                                 float eps) {
    return tsh::block_impl(backend, rulebook, h, conv_w, conv_b, gamma, beta, mlp0_w, mlp0_b, mlp2_w, mlp2_b, out, n,
                           c, eps);
}

trellis_status trellis_sparse_hip_conv_norm(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                            const trellis_sparse_buffer * feats, const float * weight,
                                            const float * bias, const float * gamma, const float * beta, float eps,
                                            int silu, trellis_sparse_buffer * out, int64_t n, int ci, int co) {
    return tsh::conv_norm_impl(backend, rulebook, feats, weight, bias, gamma, beta, eps, silu, out, n, ci, co);
}

trellis_status trellis_sparse_hip_conv_add(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                           const trellis_sparse_buffer * feats, const float * weight,
                                           const float * bias, const trellis_sparse_buffer * residual,
                                           trellis_sparse_buffer * out, int64_t n, int ci, int co) {
    return tsh::conv_add_impl(backend, rulebook, feats, weight, bias, residual, out, n, ci, co);
}

trellis_status trellis_sparse_hip_profile_enable(trellis_sparse_backend * backend, int enable) {
    if (backend == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    tsh::as_backend(backend)->profiling = enable != 0;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_profile_read(trellis_sparse_backend * backend, trellis_sparse_hip_stage_times * out,
                                               int reset) {
    if (backend == nullptr || out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    const hipError_t err = hipStreamSynchronize(be->stream);
    if (err != hipSuccess) return tsh::hip_status(be, err, "profile_read");
    for (auto & m : be->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, m.a, m.b) == hipSuccess) {
            be->times.ms[m.stage] += ms;
            be->times.launches[m.stage] += 1;
        } else {
            (void) hipGetLastError();
        }
        be->spare_events.push_back(m.a);
        be->spare_events.push_back(m.b);
    }
    be->pending.clear();
    *out = be->times;
    if (reset) be->times = trellis_sparse_hip_stage_times{};
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_event_record(trellis_sparse_backend * backend, int slot) {
    if (backend == nullptr || slot < 0 || slot >= 16) return TRELLIS_STATUS_INVALID_ARGUMENT;
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    if (be->user_events[slot] == nullptr) {
        const hipError_t err = hipEventCreate(&be->user_events[slot]);
        if (err != hipSuccess) return tsh::hip_status(be, err, "event_create");
    }
    return tsh::hip_status(be, hipEventRecord(be->user_events[slot], be->stream), "event_record");
}

trellis_status trellis_sparse_hip_event_elapsed(trellis_sparse_backend * backend, int slot_a, int slot_b, float * ms) {
    if (backend == nullptr || ms == nullptr || slot_a < 0 || slot_a >= 16 || slot_b < 0 || slot_b >= 16) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    Backend * be = tsh::as_backend(backend);
    tsh::select_device(be);
    if (be->user_events[slot_a] == nullptr || be->user_events[slot_b] == nullptr) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    hipError_t err = hipEventSynchronize(be->user_events[slot_b]);
    if (err == hipSuccess) err = hipEventElapsedTime(ms, be->user_events[slot_a], be->user_events[slot_b]);
    return tsh::hip_status(be, err, "event_elapsed");
}

}  // extern "C"
