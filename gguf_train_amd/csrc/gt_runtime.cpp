// Runtime of libgt_attn.so: errors, device discovery, per-thread streams, the device memory
// pool, storage/handle lifecycle, host<->device copies and DLPack export.
//
// Mirrors the lifecycle half of the reference ABI (csrc/gt_core.cpp:457-1087) with HIP device
// memory instead of ggml backend buffers.

#include "gt_half.h"
#include "gt_internal.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <vector>

// ---------------------------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------------------------

static thread_local std::string t_last_error;

void gt_set_error(const std::string &msg) { t_last_error = msg; }

bool gt_hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    gt_set_error(std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

extern "C" const char *gt_last_error(void) { return t_last_error.c_str(); }
extern "C" void gt_clear_error(void) { t_last_error.clear(); }
extern "C" void gt_set_last_error(const char *msg) { t_last_error = msg ? msg : ""; }

// ---------------------------------------------------------------------------------------------
// init / devices / streams
// ---------------------------------------------------------------------------------------------

static std::once_flag g_init_once;
static int g_device_count = 0;

// Fingerprint of the sources this library was built from (the build passes it; the Python
// loader compares it with the sources beside the library).
#ifndef GT_SOURCE_HASH
#define GT_SOURCE_HASH "unknown"
#endif
extern "C" const char *gt_source_hash(void) { return GT_SOURCE_HASH; }

extern "C" void gt_init(void) {
    std::call_once(g_init_once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        (void)hipGetLastError();
        g_device_count = n;
    });
}

bool gt_device_ok(int idx) {
    gt_init();
    if (g_device_count <= 0) {
        gt_set_error("no HIP device is available (libgt_attn computes on the GPU only)");
        return false;
    }
    if (idx < 0 || idx >= g_device_count) {
        gt_set_error("HIP device index " + std::to_string(idx) + " is out of range (" +
                     std::to_string(g_device_count) + " devices)");
        return false;
    }
    return gt_hip_check(hipSetDevice(idx), "hipSetDevice");
}

static thread_local hipStream_t t_stream = nullptr;

hipStream_t gt_stream() { return t_stream; }
extern "C" void gt_set_stream(void *stream) { t_stream = (hipStream_t)stream; }
extern "C" void *gt_get_stream(void) { return (void *)t_stream; }

// One uncached buffer per (device, stream), grown on demand.  The decode kernels' in-kernel
// split merge is correct only in this memory (hipDeviceMallocUncached: no XCD's L2 holds the
// partials or the counters; see decode_merge.h).  The kernels leave every counter at zero, so a
// buffer is zeroed only when it is created.  Uncached memory is never freed while the process
// runs (memory allocated after such a free has read wrong values on these GPUs, and launches in
// flight may still use a replaced buffer), so the footprint is bounded instead:
//   - a buffer grows at least twofold, to at most kMaxWorkspaceBytes; a request beyond that
//     returns false (the launch then merges its splits with a second kernel over pooled memory);
//   - a replaced buffer stays listed in `retired` (held, not lost), so one stream holds less
//     than 2 x kMaxWorkspaceBytes in all (the sizes form a doubling series);
//   - at most kMaxWorkspaceStreams streams per device get a workspace; calls on further streams
//     return false.
// Per device that is at most 16 x 2 x 64 MiB; the benchmark's decode shapes need 1 MiB each.
bool gt_decode_workspace(int dev, hipStream_t s, int64_t n_counters, size_t part_bytes, gt_decode_ws &ws) {
    constexpr size_t kMaxWorkspaceStreams = 16;
    constexpr size_t kMaxWorkspaceBytes = (size_t)64 << 20;
    static std::mutex mu;
    struct Buf {
        char *p = nullptr;
        int64_t counters = 0;
        size_t parts = 0;
    };
    static std::map<std::pair<int, hipStream_t>, Buf> bufs;
    static std::map<int, size_t> streams_of;  // workspaces per device
    static std::vector<char *> retired;       // replaced buffers, held until the process ends
    const size_t cbytes_of = 256;  // granule of the counter area
    auto cbytes = [&](int64_t n) { return ((size_t)n * sizeof(int) + cbytes_of - 1) / cbytes_of * cbytes_of; };
    if (n_counters < 0 || cbytes(n_counters) + part_bytes > kMaxWorkspaceBytes) return false;
    std::lock_guard<std::mutex> lock(mu);
    auto found = bufs.find({dev, s});
    if (found == bufs.end()) {
        if (streams_of[dev] >= kMaxWorkspaceStreams) return false;
        ++streams_of[dev];
        found = bufs.emplace(std::make_pair(dev, s), Buf{}).first;
    }
    Buf &e = found->second;
    if (!e.p || e.counters < n_counters || e.parts < part_bytes) {
        Buf nb;
        nb.counters = std::max<int64_t>({n_counters, 2 * e.counters, 4096});
        nb.parts = std::max<size_t>({part_bytes, 2 * e.parts, (size_t)1 << 20});
        // the doubling stops at the cap (the request itself fits, checked above)
        while (cbytes(nb.counters) + nb.parts > kMaxWorkspaceBytes) {
            if (nb.parts > part_bytes) nb.parts = std::max(part_bytes, nb.parts / 2);
            else nb.counters = std::max(n_counters, nb.counters / 2);
        }
        if (hipExtMallocWithFlags((void **)&nb.p, cbytes(nb.counters) + nb.parts, hipDeviceMallocUncached) !=
                hipSuccess ||
            !nb.p) {
            (void)hipGetLastError();
            return false;
        }
        if (gt_launch_fill_zero(nb.p, (int64_t)cbytes(nb.counters), s) != hipSuccess) {
            (void)hipGetLastError();
            retired.push_back(nb.p);  // held (never freed), unused
            return false;
        }
        if (e.p) retired.push_back(e.p);
        e = nb;
    }
    ws.counters = (int *)e.p;
    ws.parts = e.p + cbytes(e.counters);
    return true;
}

extern "C" int gt_device_count(int device_type) {
    gt_init();
    if (device_type == GT_DEV_CPU) return 1;
    if (device_type == GT_DEV_CUDA) return g_device_count;
    return 0;
}

extern "C" void gt_device_name(int device_type, int idx, char *buf, int buf_len) {
    if (!buf || buf_len <= 0) return;
    buf[0] = 0;
    if (device_type == GT_DEV_CPU) {
        snprintf(buf, buf_len, "CPU");
        return;
    }
    if (device_type != GT_DEV_CUDA || !gt_device_ok(idx)) return;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, idx) == hipSuccess) snprintf(buf, buf_len, "%s (%s)", p.name, p.gcnArchName);
}

extern "C" void gt_device_memory(int device_type, int idx, size_t *free_bytes, size_t *total_bytes) {
    size_t f = 0, t = 0;
    if (device_type == GT_DEV_CUDA && gt_device_ok(idx)) (void)hipMemGetInfo(&f, &t);
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
}

extern "C" void gt_synchronize(int device_type, int idx) {
    if (device_type != GT_DEV_CUDA || !gt_device_ok(idx)) return;
    (void)hipDeviceSynchronize();
}

// ---------------------------------------------------------------------------------------------
// dtype helpers
// ---------------------------------------------------------------------------------------------

size_t gt_elem_bytes(int dtype) {
    switch (dtype) {
        case GT_F32: return 4;
        case GT_F16: return 2;
        case GT_BF16: return 2;
        case GT_F64: return 8;
        case GT_I8: return 1;
        case GT_U8: return 1;
        case GT_I16: return 2;
        case GT_I32: return 4;
        case GT_I64: return 8;
        case GT_BOOL: return 1;
        case GT_C64: return 8;
        case GT_C128: return 16;
        default: return 0;
    }
}

size_t gt_dtype_nbytes(int dtype, int64_t numel) {
    if (dtype == GT_Q8_0) return (size_t)((numel + 31) / 32) * 34;
    return (size_t)numel * gt_elem_bytes(dtype);
}

const char *gt_dtype_name(int dtype) {
    switch (dtype) {
        case GT_F32: return "float32";
        case GT_F16: return "float16";
        case GT_BF16: return "bfloat16";
        case GT_F64: return "float64";
        case GT_I8: return "int8";
        case GT_U8: return "uint8";
        case GT_I16: return "int16";
        case GT_I32: return "int32";
        case GT_I64: return "int64";
        case GT_BOOL: return "bool";
        case GT_C64: return "complex64";
        case GT_C128: return "complex128";
        case GT_Q8_0: return "q8_0";
        default: return "unknown";
    }
}

static bool dtype_supported(int dtype) {
    return (gt_elem_bytes(dtype) > 0 && dtype != GT_C64 && dtype != GT_C128) || dtype == GT_Q8_0;
}

extern "C" size_t gt_tensor_elem_size(int dtype) { return gt_elem_bytes(dtype); }

void gt_default_strides(int ndim, const int64_t *shape, int64_t *strides) {
    int64_t s = 1;
    for (int i = ndim - 1; i >= 0; --i) {
        strides[i] = s;
        s *= std::max<int64_t>(shape[i], 1);
    }
}

bool gt_is_dense(const gt_tensor *t) {
    if (t->numel == 0 || t->ndim == 0) return true;
    int64_t expected = 1;
    for (int i = t->ndim - 1; i >= 0; --i) {
        if (t->shape[i] != 1) {
            if (t->strides[i] != expected) return false;
            expected *= t->shape[i];
        }
    }
    return true;
}

void *gt_data(const gt_tensor *t) {
    if (!t || !t->storage || !t->storage->ptr) return nullptr;
    if (gt_is_quantized(t->dtype)) return t->storage->ptr;  // quantized tensors are whole storages
    return (char *)t->storage->ptr + (size_t)t->offset * gt_elem_bytes(t->dtype);
}

// ---------------------------------------------------------------------------------------------
// external-memory release queue (csrc/gt_core.cpp:524-552)
// ---------------------------------------------------------------------------------------------

namespace {
struct ExternalQueue {
    std::mutex mu;
    std::vector<uint64_t> tokens;
};
ExternalQueue &external_queue() {
    static ExternalQueue *q = new ExternalQueue();  // never destroyed: storages may die at exit
    return *q;
}
}  // namespace

extern "C" int64_t gt_external_released(uint64_t *tokens, int64_t capacity) {
    if (!tokens || capacity <= 0) return 0;
    ExternalQueue &q = external_queue();
    std::lock_guard<std::mutex> lock(q.mu);
    const int64_t n = std::min<int64_t>(capacity, (int64_t)q.tokens.size());
    for (int64_t i = 0; i < n; ++i) tokens[i] = q.tokens[(size_t)i];
    q.tokens.erase(q.tokens.begin(), q.tokens.begin() + n);
    return n;
}

// ---------------------------------------------------------------------------------------------
// device memory pool
//
// Blocks freed by a storage go back to a free list keyed by size and are reused by a later
// allocation on the same device and stream: work on one stream runs in order, so a block is
// never handed out while a kernel that used it can still be running.  hipFree (which waits
// for the whole device) only runs when hipMalloc fails, after which the cache is emptied and
// the allocation retried.
// ---------------------------------------------------------------------------------------------

namespace {
struct PoolBlock {
    void *ptr;
    size_t size;
    int dev;
    hipStream_t stream;
};

class DevicePool {
  public:
    void *alloc(size_t want, int dev, hipStream_t stream, size_t *got) {
        const size_t size = round_size(want);
        {
            std::lock_guard<std::mutex> lock(mu_);
            // best fit among blocks no larger than twice the request (bounded waste)
            for (auto it = free_.lower_bound(size); it != free_.end() && it->first <= 2 * size; ++it) {
                if (it->second.dev == dev && it->second.stream == stream) {
                    void *p = it->second.ptr;
                    *got = it->second.size;
                    cached_ -= it->second.size;
                    free_.erase(it);
                    return p;
                }
            }
        }
        void *p = nullptr;
        if (hipMalloc(&p, size) != hipSuccess) {
            (void)hipGetLastError();
            empty_cache();
            if (hipMalloc(&p, size) != hipSuccess) {
                (void)hipGetLastError();
                return nullptr;
            }
        }
        *got = size;
        return p;
    }

    void release(void *p, size_t size, int dev, hipStream_t stream) {
        std::lock_guard<std::mutex> lock(mu_);
        free_.emplace(size, PoolBlock{p, size, dev, stream});
        cached_ += size;
    }

    void empty_cache() {
        std::multimap<size_t, PoolBlock> blocks;
        {
            std::lock_guard<std::mutex> lock(mu_);
            blocks.swap(free_);
            cached_ = 0;
        }
        if (blocks.empty()) return;
        (void)hipDeviceSynchronize();
        for (auto &kv : blocks) (void)hipFree(kv.second.ptr);
    }

  private:
    static size_t round_size(size_t n) {
        if (n == 0) n = 1;
        if (n <= ((size_t)1 << 20)) return (n + 511) & ~(size_t)511;
        const size_t g = (size_t)2 << 20;
        return (n + g - 1) / g * g;
    }
    std::mutex mu_;
    std::multimap<size_t, PoolBlock> free_;
    size_t cached_ = 0;
};

DevicePool &pool() {
    static DevicePool *p = new DevicePool();  // never destroyed: storages may die at exit
    return *p;
}

// Failure injection for the error paths: while GT_ATTN_FAIL_ALLOC is set to a non-zero value
// every storage allocation fails as if memory were exhausted.
bool injected_alloc_failure() {
    const char *v = std::getenv("GT_ATTN_FAIL_ALLOC");
    return v && v[0] && std::strcmp(v, "0") != 0;
}
}  // namespace

gt_storage::~gt_storage() {
    if (!ptr) return;
    if (kind == GT_STORE_HOST) {
        std::free(ptr);
    } else if (kind == GT_STORE_DEVICE) {
        pool().release(ptr, capacity, device_index, stream);
    } else if (token) {
        ExternalQueue &q = external_queue();
        std::lock_guard<std::mutex> lock(q.mu);
        q.tokens.push_back(token);
    }
}

static std::shared_ptr<gt_storage> alloc_storage(size_t nbytes, int64_t numel, int device_type, int device_index) {
    if (injected_alloc_failure()) {
        gt_set_error("out of memory: storage allocation of " + std::to_string(nbytes) +
                     " bytes failed (GT_ATTN_FAIL_ALLOC is set)");
        return nullptr;
    }
    auto st = std::make_shared<gt_storage>();
    st->nbytes = nbytes;
    st->numel = numel;
    st->device_type = device_type;
    st->device_index = device_index;
    if (device_type == GT_DEV_CPU) {
        const size_t cap = (std::max<size_t>(nbytes, 1) + 63) & ~(size_t)63;
        st->ptr = std::aligned_alloc(64, cap);
        st->capacity = cap;
        st->kind = GT_STORE_HOST;
        if (!st->ptr) {
            gt_set_error("out of host memory allocating " + std::to_string(nbytes) + " bytes");
            return nullptr;
        }
        return st;
    }
    if (device_type != GT_DEV_CUDA) {
        gt_set_error("device type " + std::to_string(device_type) + " is not supported (CPU or HIP only)");
        return nullptr;
    }
    if (!gt_device_ok(device_index)) return nullptr;
    st->kind = GT_STORE_DEVICE;
    st->stream = gt_stream();
    st->ptr = pool().alloc(nbytes, device_index, st->stream, &st->capacity);
    if (!st->ptr) {
        gt_set_error("out of device memory allocating " + std::to_string(nbytes) + " bytes");
        return nullptr;
    }
    return st;
}

bool gt_scratch_alloc(gt_scratch &s, size_t nbytes, int dev) {
    s.st = alloc_storage(nbytes, (int64_t)nbytes, GT_DEV_CUDA, dev);
    return (bool)s.st;
}

gt_tensor *gt_new_tensor(int ndim, const int64_t *shape, int dtype, int device_type, int device_index) {
    gt_init();
    if (ndim < 0 || ndim > GT_MAX_DIMS || (ndim > 0 && !shape)) {
        gt_set_error("Invalid ndim");
        return nullptr;
    }
    for (int i = 0; i < ndim; ++i) {
        if (shape[i] < 0) {
            gt_set_error("Negative dimension size");
            return nullptr;
        }
    }
    if (!dtype_supported(dtype)) {
        gt_set_error(std::string("dtype ") + std::to_string(dtype) + " (" + gt_dtype_name(dtype) +
                     ") is not supported by libgt_attn");
        return nullptr;
    }
    const int64_t numel = gt_numel_of(ndim, shape);
    auto st = alloc_storage(gt_dtype_nbytes(dtype, numel), numel, device_type, device_index);
    if (!st) return nullptr;
    auto *t = new gt_tensor();
    t->ndim = ndim;
    for (int i = 0; i < ndim; ++i) t->shape[i] = shape[i];
    gt_default_strides(ndim, t->shape, t->strides);
    t->numel = numel;
    t->dtype = dtype;
    t->device_type = device_type;
    t->device_index = device_index;
    t->storage = std::move(st);
    return t;
}

// ---------------------------------------------------------------------------------------------
// lifecycle ABI
// ---------------------------------------------------------------------------------------------

extern "C" gt_tensor *gt_tensor_empty(int ndim, const int64_t *shape, int dtype, int device_type, int device_index) {
    return gt_new_tensor(ndim, shape, dtype, device_type, device_index);
}

extern "C" gt_tensor *gt_tensor_from_data(int ndim, const int64_t *shape, int dtype, int device_type,
                                          int device_index, const void *data, size_t nbytes) {
    gt_tensor *t = gt_new_tensor(ndim, shape, dtype, device_type, device_index);
    if (!t) return nullptr;
    if (data && nbytes > 0 && t->numel > 0 && gt_tensor_copy_from_host(t, data, nbytes) != 0) {
        gt_tensor_free(t);
        return nullptr;
    }
    return t;
}

// Validation shared by the two borrowed-memory constructors (csrc/gt_core.cpp:554-610).
static bool check_external(const char *who, int ndim, const int64_t *shape, const int64_t *strides, int dtype,
                           const void *data, uint64_t token, int64_t *numel_out, int64_t *extent_out) {
    if (ndim < 0 || ndim > GT_MAX_DIMS || (ndim > 0 && (!shape || !strides))) {
        gt_set_error(std::string(who) + ": invalid ndim");
        return false;
    }
    if (!data || token == 0) {
        gt_set_error(std::string(who) + ": a data pointer and a non-zero token are required");
        return false;
    }
    const size_t es = gt_elem_bytes(dtype);
    if (es == 0 || !dtype_supported(dtype) || gt_is_quantized(dtype)) {
        gt_set_error(std::string(who) + ": unsupported dtype");
        return false;
    }
    if ((uintptr_t)data % es != 0) {
        gt_set_error(std::string(who) + ": the data pointer is not aligned for the element type");
        return false;
    }
    const int64_t limit = std::numeric_limits<int64_t>::max() / (int64_t)(2 * es);
    int64_t extent = 1, numel = 1;
    for (int i = 0; i < ndim; ++i) {
        if (shape[i] <= 0) {
            gt_set_error(std::string(who) + ": every dimension must have at least one element");
            return false;
        }
        if (strides[i] < 0) {
            gt_set_error(std::string(who) + ": negative strides are not supported");
            return false;
        }
        const int64_t steps = shape[i] - 1;
        if (steps > 0 && strides[i] > (limit - extent) / steps) {
            gt_set_error(std::string(who) + ": the array is too large");
            return false;
        }
        extent += steps * strides[i];
        if (shape[i] > limit / numel) {
            gt_set_error(std::string(who) + ": the array is too large");
            return false;
        }
        numel *= shape[i];
    }
    *numel_out = numel;
    *extent_out = extent;
    return true;
}

static gt_tensor *make_external(int ndim, const int64_t *shape, const int64_t *strides, int dtype, void *data,
                                uint64_t token, int device_type, int device_index, int64_t numel, int64_t extent) {
    auto st = std::make_shared<gt_storage>();
    st->ptr = data;
    st->numel = extent;
    st->nbytes = (size_t)extent * gt_elem_bytes(dtype);
    st->device_type = device_type;
    st->device_index = device_index;
    st->kind = GT_STORE_EXTERNAL;
    st->token = token;
    auto *t = new gt_tensor();
    t->ndim = ndim;
    for (int i = 0; i < ndim; ++i) {
        t->shape[i] = shape[i];
        t->strides[i] = strides[i];
    }
    t->numel = numel;
    t->dtype = dtype;
    t->device_type = device_type;
    t->device_index = device_index;
    t->storage = std::move(st);
    return t;
}

extern "C" gt_tensor *gt_tensor_from_external(int ndim, const int64_t *shape, const int64_t *strides, int dtype,
                                              void *data, uint64_t token) {
    gt_init();
    int64_t numel = 0, extent = 0;
    if (!check_external("from_external", ndim, shape, strides, dtype, data, token, &numel, &extent)) return nullptr;
    return make_external(ndim, shape, strides, dtype, data, token, GT_DEV_CPU, 0, numel, extent);
}

extern "C" gt_tensor *gt_tensor_from_device_ptr(int ndim, const int64_t *shape, const int64_t *strides, int dtype,
                                                int device_index, void *data, uint64_t token) {
    gt_init();
    int64_t numel = 0, extent = 0;
    if (dtype == GT_Q8_0) {
        // quantized blocks: a dense row-major logical shape over whole 34-byte blocks
        int64_t want[GT_MAX_DIMS];
        if (ndim < 1 || ndim > GT_MAX_DIMS || !shape || !strides || !data || token == 0) {
            gt_set_error("from_device_ptr: invalid arguments");
            return nullptr;
        }
        gt_default_strides(ndim, shape, want);
        numel = gt_numel_of(ndim, shape);
        for (int i = 0; i < ndim; ++i) {
            if (shape[i] <= 0 || strides[i] != want[i]) {
                gt_set_error("from_device_ptr: a q8_0 tensor must be dense with every dimension non-empty");
                return nullptr;
            }
        }
        if (numel % 32 != 0 || (uintptr_t)data % 2 != 0) {
            gt_set_error("from_device_ptr: a q8_0 tensor holds whole 32-value blocks at a 2-byte aligned address");
            return nullptr;
        }
        if (!gt_device_ok(device_index)) return nullptr;
        gt_tensor *t = make_external(ndim, shape, strides, GT_F16, data, token, GT_DEV_CUDA, device_index, numel, numel);
        t->dtype = GT_Q8_0;
        t->storage->nbytes = gt_dtype_nbytes(GT_Q8_0, numel);
        return t;
    }
    if (!check_external("from_device_ptr", ndim, shape, strides, dtype, data, token, &numel, &extent)) return nullptr;
    if (!gt_device_ok(device_index)) return nullptr;
    return make_external(ndim, shape, strides, dtype, data, token, GT_DEV_CUDA, device_index, numel, extent);
}

extern "C" gt_tensor *gt_tensor_view(const gt_tensor *t, int ndim, const int64_t *shape, const int64_t *strides,
                                     int64_t offset) {
    if (!t || ndim < 0 || ndim > GT_MAX_DIMS || (ndim > 0 && (!shape || !strides))) {
        gt_set_error("Invalid view arguments");
        return nullptr;
    }
    if (gt_is_quantized(t->dtype)) {
        gt_set_error("view: quantized tensors cannot be viewed");
        return nullptr;
    }
    bool empty = false;
    int64_t lo = offset, hi = offset;
    for (int i = 0; i < ndim; ++i) {
        if (shape[i] < 0) {
            gt_set_error("view: negative dimension size " + std::to_string(shape[i]));
            return nullptr;
        }
        if (shape[i] == 0) empty = true;
        const int64_t span = (shape[i] - 1) * strides[i];
        if (span < 0) lo += span; else hi += span;
    }
    if (!empty && t->storage && (lo < 0 || hi >= t->storage->numel)) {
        gt_set_error("view: elements " + std::to_string(lo) + ".." + std::to_string(hi) +
                     " lie outside the storage of " + std::to_string(t->storage->numel) + " elements");
        return nullptr;
    }
    auto *out = new gt_tensor();
    out->ndim = ndim;
    for (int i = 0; i < ndim; ++i) {
        out->shape[i] = shape[i];
        out->strides[i] = strides[i];
    }
    out->offset = offset;
    out->numel = gt_numel_of(ndim, shape);
    out->dtype = t->dtype;
    out->device_type = t->device_type;
    out->device_index = t->device_index;
    out->storage = t->storage;
    return out;
}

extern "C" void gt_tensor_free(gt_tensor *t) { delete t; }

extern "C" int gt_tensor_ndim(const gt_tensor *t) { return t ? t->ndim : 0; }
extern "C" void gt_tensor_shape(const gt_tensor *t, int64_t *out) {
    if (t && out) for (int i = 0; i < t->ndim; ++i) out[i] = t->shape[i];
}
extern "C" void gt_tensor_strides(const gt_tensor *t, int64_t *out) {
    if (t && out) for (int i = 0; i < t->ndim; ++i) out[i] = t->strides[i];
}
extern "C" int64_t gt_tensor_offset(const gt_tensor *t) { return t ? t->offset : 0; }
extern "C" int64_t gt_tensor_numel(const gt_tensor *t) { return t ? t->numel : 0; }
extern "C" int gt_tensor_dtype(const gt_tensor *t) { return t ? t->dtype : GT_F32; }
extern "C" int gt_tensor_device_type(const gt_tensor *t) { return t ? t->device_type : GT_DEV_CPU; }
extern "C" int gt_tensor_device_index(const gt_tensor *t) { return t ? t->device_index : 0; }
extern "C" int gt_tensor_is_contiguous(const gt_tensor *t) { return (t && gt_is_dense(t)) ? 1 : 0; }
extern "C" uint64_t gt_tensor_data_ptr(const gt_tensor *t) { return (uint64_t)(uintptr_t)gt_data(t); }
extern "C" size_t gt_tensor_storage_nbytes(const gt_tensor *t) { return (t && t->storage) ? t->storage->nbytes : 0; }
extern "C" size_t gt_tensor_nbytes(const gt_tensor *t) {
    if (!t) return 0;
    return gt_dtype_nbytes(t->dtype, t->numel);
}

// ---------------------------------------------------------------------------------------------
// element conversion on the host (host tensors only; device tensors use gt_launch_convert)
// ---------------------------------------------------------------------------------------------

static double host_read(const void *p, int dtype, int64_t i) {
    switch (dtype) {
        case GT_F32: return ((const float *)p)[i];
        case GT_F64: return ((const double *)p)[i];
        case GT_F16: return gt::f16_to_f32(((const uint16_t *)p)[i]);
        case GT_BF16: return gt::bf16_to_f32(((const uint16_t *)p)[i]);
        case GT_I8: return ((const int8_t *)p)[i];
        case GT_U8: return ((const uint8_t *)p)[i];
        case GT_I16: return ((const int16_t *)p)[i];
        case GT_I32: return ((const int32_t *)p)[i];
        case GT_I64: return (double)((const int64_t *)p)[i];
        case GT_BOOL: return ((const uint8_t *)p)[i] ? 1.0 : 0.0;
        default: return 0.0;
    }
}

static void host_write(void *p, int dtype, int64_t i, double v) {
    switch (dtype) {
        case GT_F32: ((float *)p)[i] = (float)v; break;
        case GT_F64: ((double *)p)[i] = v; break;
        case GT_F16: ((uint16_t *)p)[i] = gt::f32_to_f16((float)v); break;
        case GT_BF16: ((uint16_t *)p)[i] = gt::f32_to_bf16((float)v); break;
        case GT_I8: ((int8_t *)p)[i] = (int8_t)v; break;
        case GT_U8: ((uint8_t *)p)[i] = (uint8_t)v; break;
        case GT_I16: ((int16_t *)p)[i] = (int16_t)v; break;
        case GT_I32: ((int32_t *)p)[i] = (int32_t)v; break;
        case GT_I64: ((int64_t *)p)[i] = (int64_t)v; break;
        case GT_BOOL: ((uint8_t *)p)[i] = v != 0.0 ? 1 : 0; break;
        default: break;
    }
}

static int64_t strided_offset(const int64_t *shape, const int64_t *strides, int ndim, int64_t linear) {
    int64_t off = 0;
    for (int d = ndim - 1; d >= 0; --d) {
        const int64_t c = linear % shape[d];
        linear /= shape[d];
        off += c * strides[d];
    }
    return off;
}

// Host strided -> host strided element copy with conversion (same shape).
static void host_convert(const gt_tensor *src, gt_tensor *dst) {
    const char *sb = (const char *)src->storage->ptr;
    char *db = (char *)dst->storage->ptr;
    const bool same = src->dtype == dst->dtype;
    const size_t es = gt_elem_bytes(src->dtype);
    for (int64_t i = 0; i < src->numel; ++i) {
        const int64_t so = src->offset + strided_offset(src->shape, src->strides, src->ndim, i);
        const int64_t doff = dst->offset + strided_offset(dst->shape, dst->strides, dst->ndim, i);
        if (same) {
            std::memcpy(db + doff * es, sb + so * es, es);
        } else if (dst->dtype == GT_I64 && src->dtype == GT_I64) {
            ((int64_t *)db)[doff] = ((const int64_t *)sb)[so];
        } else {
            host_write(db, dst->dtype, doff, host_read(sb, src->dtype, so));
        }
    }
}

static gt_layout layout_of(const gt_tensor *t) {
    gt_layout l{};
    l.ndim = t->ndim;
    for (int i = 0; i < t->ndim; ++i) {
        l.shape[i] = t->shape[i];
        l.strides[i] = t->strides[i];
    }
    return l;
}

static gt_layout dense_layout(const gt_tensor *t) {
    gt_layout l = layout_of(t);
    gt_default_strides(l.ndim, l.shape, l.strides);
    return l;
}

// Device strided -> device strided copy with conversion (same shape), enqueued on the stream.
static bool device_convert(const gt_tensor *src, gt_tensor *dst) {
    if (src->numel == 0) return true;
    if (!gt_device_ok(dst->device_index)) return false;
    return gt_hip_check(gt_launch_convert(gt_data(src), src->dtype, layout_of(src), gt_data(dst), dst->dtype,
                                          layout_of(dst), src->numel, gt_stream()),
                        "convert kernel");
}

// The span [first, last] of elements a strided host tensor reaches, for staging to the device.
static void element_span(const gt_tensor *t, int64_t *lo, int64_t *hi) {
    *lo = t->offset;
    *hi = t->offset;
    for (int i = 0; i < t->ndim; ++i) {
        if (t->shape[i] <= 0) continue;
        const int64_t s = (t->shape[i] - 1) * t->strides[i];
        if (s < 0) *lo += s; else *hi += s;
    }
}

gt_tensor *gt_to_device_dense(const gt_tensor *t, int dev, int dtype) {
    if (dtype < 0) dtype = t->dtype;
    if (gt_is_quantized(t->dtype) || gt_is_quantized(dtype)) {
        if (t->dtype != dtype) {
            gt_set_error("internal: quantized conversion requested through gt_to_device_dense");
            return nullptr;
        }
        gt_tensor *out = gt_new_tensor(t->ndim, t->shape, t->dtype, GT_DEV_CUDA, dev);
        if (!out) return nullptr;
        const size_t nb = gt_dtype_nbytes(t->dtype, t->numel);
        const hipMemcpyKind kind = t->device_type == GT_DEV_CPU ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
        if (nb && !gt_hip_check(hipMemcpyAsync(out->storage->ptr, t->storage->ptr, nb, kind, gt_stream()),
                                "hipMemcpyAsync")) {
            gt_tensor_free(out);
            return nullptr;
        }
        if (kind == hipMemcpyHostToDevice && !gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize")) {
            gt_tensor_free(out);
            return nullptr;
        }
        return out;
    }
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, dtype, GT_DEV_CUDA, dev);
    if (!out) return nullptr;
    if (t->numel == 0) return out;
    if (t->device_type == GT_DEV_CUDA) {
        if (!device_convert(t, out)) {
            gt_tensor_free(out);
            return nullptr;
        }
        return out;
    }
    // host source: move the reachable span as raw bytes, then gather/convert on the device
    int64_t lo, hi;
    element_span(t, &lo, &hi);
    const size_t es = gt_elem_bytes(t->dtype);
    const int64_t span = hi - lo + 1;
    if (gt_is_dense(t) && t->dtype == dtype) {
        if (!gt_hip_check(hipMemcpyAsync(out->storage->ptr, (const char *)t->storage->ptr + (size_t)t->offset * es,
                                         (size_t)t->numel * es, hipMemcpyHostToDevice, gt_stream()),
                          "hipMemcpyAsync") ||
            !gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize")) {
            gt_tensor_free(out);
            return nullptr;
        }
        return out;
    }
    gt_scratch stage;
    if (!gt_scratch_alloc(stage, (size_t)span * es, dev)) {
        gt_tensor_free(out);
        return nullptr;
    }
    if (!gt_hip_check(hipMemcpyAsync(stage.ptr(), (const char *)t->storage->ptr + (size_t)lo * es, (size_t)span * es,
                                     hipMemcpyHostToDevice, gt_stream()),
                      "hipMemcpyAsync") ||
        !gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize")) {
        gt_tensor_free(out);
        return nullptr;
    }
    gt_layout sl = layout_of(t);
    const char *base = (const char *)stage.ptr() + (size_t)(t->offset - lo) * es;
    if (!gt_hip_check(gt_launch_convert(base, t->dtype, sl, out->storage->ptr, dtype, dense_layout(out), t->numel,
                                        gt_stream()),
                      "convert kernel")) {
        gt_tensor_free(out);
        return nullptr;
    }
    return out;
}

bool gt_copy_device_to_host(gt_tensor *dst, const gt_tensor *src) {
    const size_t nb = gt_dtype_nbytes(src->dtype, src->numel);
    if (nb == 0) return true;
    if (!gt_device_ok(src->device_index)) return false;
    return gt_hip_check(hipMemcpyAsync(gt_data(dst), gt_data(src), nb, hipMemcpyDeviceToHost, gt_stream()),
                        "hipMemcpyAsync") &&
           gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize");
}

gt_tensor *gt_deliver(gt_tensor *dev_t, bool to_host) {
    if (!dev_t || !to_host) return dev_t;
    gt_tensor *h = gt_new_tensor(dev_t->ndim, dev_t->shape, dev_t->dtype, GT_DEV_CPU, 0);
    if (h && !gt_copy_device_to_host(h, dev_t)) {
        gt_tensor_free(h);
        h = nullptr;
    }
    gt_tensor_free(dev_t);
    return h;
}

extern "C" int gt_tensor_copy_to_host(const gt_tensor *t, void *dst, size_t dst_bytes) {
    if (!t || !dst) {
        gt_set_error("copy_to_host: NULL argument");
        return -1;
    }
    if (t->numel == 0) return 0;
    const size_t nb = gt_dtype_nbytes(t->dtype, t->numel);
    if (dst_bytes < nb) {
        gt_set_error("copy_to_host: destination holds " + std::to_string(dst_bytes) + " bytes, " +
                     std::to_string(nb) + " needed");
        return -1;
    }
    if (t->device_type == GT_DEV_CPU) {
        if (gt_is_quantized(t->dtype) || gt_is_dense(t)) {
            std::memcpy(dst, gt_data(t), nb);
            return 0;
        }
        gt_tensor tmp;
        tmp.ndim = t->ndim;
        for (int i = 0; i < t->ndim; ++i) tmp.shape[i] = t->shape[i];
        gt_default_strides(tmp.ndim, tmp.shape, tmp.strides);
        tmp.numel = t->numel;
        tmp.dtype = t->dtype;
        tmp.storage = std::make_shared<gt_storage>();
        tmp.storage->ptr = dst;
        tmp.storage->kind = GT_STORE_EXTERNAL;  // token 0: nothing reported
        host_convert(t, &tmp);
        return 0;
    }
    if (!gt_device_ok(t->device_index)) return -1;
    if (gt_is_quantized(t->dtype) || gt_is_dense(t)) {
        if (!gt_hip_check(hipMemcpyAsync(dst, gt_data(t), nb, hipMemcpyDeviceToHost, gt_stream()), "hipMemcpyAsync") ||
            !gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize"))
            return -1;
        return 0;
    }
    gt_tensor *dense = gt_to_device_dense(t, t->device_index, -1);
    if (!dense) return -1;
    const int rc = (gt_hip_check(hipMemcpyAsync(dst, gt_data(dense), nb, hipMemcpyDeviceToHost, gt_stream()),
                                 "hipMemcpyAsync") &&
                    gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize"))
                       ? 0
                       : -1;
    gt_tensor_free(dense);
    return rc;
}

extern "C" int gt_tensor_copy_from_host(gt_tensor *t, const void *src, size_t src_bytes) {
    if (!t || !src) {
        gt_set_error("copy_from_host: NULL argument");
        return -1;
    }
    if (t->numel == 0) return 0;
    const size_t nb = gt_dtype_nbytes(t->dtype, t->numel);
    if (src_bytes < nb) {
        gt_set_error("copy_from_host: source holds " + std::to_string(src_bytes) + " bytes, " + std::to_string(nb) +
                     " needed");
        return -1;
    }
    const bool dense = gt_is_quantized(t->dtype) || gt_is_dense(t);
    if (t->device_type == GT_DEV_CPU) {
        if (dense) {
            std::memcpy(gt_data(t), src, nb);
            return 0;
        }
        gt_tensor tmp;
        tmp.ndim = t->ndim;
        for (int i = 0; i < t->ndim; ++i) tmp.shape[i] = t->shape[i];
        gt_default_strides(tmp.ndim, tmp.shape, tmp.strides);
        tmp.numel = t->numel;
        tmp.dtype = t->dtype;
        tmp.storage = std::make_shared<gt_storage>();
        tmp.storage->ptr = const_cast<void *>(src);
        tmp.storage->kind = GT_STORE_EXTERNAL;
        host_convert(&tmp, t);
        return 0;
    }
    if (!gt_device_ok(t->device_index)) return -1;
    if (dense) {
        return (gt_hip_check(hipMemcpyAsync(gt_data(t), src, nb, hipMemcpyHostToDevice, gt_stream()), "hipMemcpyAsync") &&
                gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize"))
                   ? 0
                   : -1;
    }
    // strided device destination: stage densely, then scatter on the device
    gt_scratch stage;
    if (!gt_scratch_alloc(stage, nb, t->device_index)) return -1;
    if (!gt_hip_check(hipMemcpyAsync(stage.ptr(), src, nb, hipMemcpyHostToDevice, gt_stream()), "hipMemcpyAsync") ||
        !gt_hip_check(hipStreamSynchronize(gt_stream()), "hipStreamSynchronize"))
        return -1;
    gt_layout dl = layout_of(t);
    gt_layout sl = dense_layout(t);
    return gt_hip_check(gt_launch_convert(stage.ptr(), t->dtype, sl, gt_data(t), t->dtype, dl, t->numel, gt_stream()),
                        "convert kernel")
               ? 0
               : -1;
}

// dst <- src with dtype conversion; shapes must hold the same number of elements, or src must
// broadcast to dst from the right (as the reference's copy_, csrc/gt_core.cpp:990-1040).
extern "C" int gt_tensor_copy_inplace(gt_tensor *dst, const gt_tensor *src) {
    if (!dst || !src) {
        gt_set_error("copy_: NULL argument");
        return -1;
    }
    if (dst->numel == 0 || src->numel == 0) return 0;
    if (gt_is_quantized(dst->dtype) || gt_is_quantized(src->dtype)) {
        gt_set_error("copy_: quantized tensors are converted with gt_quantize / gt_dequantize");
        return -1;
    }
    // source view with dst's shape: same numel -> reshape of a dense copy; else broadcast strides
    gt_tensor view;
    const gt_tensor *s = src;
    gt_tensor *dense_src = nullptr;
    if (src->numel == dst->numel && !(src->ndim == dst->ndim &&
                                      std::equal(src->shape, src->shape + src->ndim, dst->shape))) {
        // element order of src, reshaped to dst's shape: needs a dense source
        if (!gt_is_dense(src)) {
            if (src->device_type == GT_DEV_CUDA) {
                dense_src = gt_to_device_dense(src, src->device_index, -1);
            } else {
                dense_src = gt_new_tensor(src->ndim, src->shape, src->dtype, GT_DEV_CPU, 0);
                if (dense_src) host_convert(src, dense_src);
            }
            if (!dense_src) return -1;
            s = dense_src;
        }
        view = *s;
        view.ndim = dst->ndim;
        for (int i = 0; i < dst->ndim; ++i) view.shape[i] = dst->shape[i];
        gt_default_strides(view.ndim, view.shape, view.strides);
        s = &view;
    } else if (src->numel != dst->numel) {
        if (src->ndim > dst->ndim) {
            gt_set_error("copy_: src has more dimensions than dst");
            return -1;
        }
        view = *src;
        view.ndim = dst->ndim;
        const int lead = dst->ndim - src->ndim;
        for (int i = 0; i < dst->ndim; ++i) {
            const int si = i - lead;
            const int64_t sz = si >= 0 ? src->shape[si] : 1;
            if (sz != 1 && sz != dst->shape[i]) {
                gt_set_error("copy_: src cannot be broadcast to dst");
                return -1;
            }
            view.shape[i] = dst->shape[i];
            view.strides[i] = (si >= 0 && sz != 1) ? src->strides[si] : 0;
        }
        view.numel = dst->numel;
        s = &view;
    }
    int rc = 0;
    gt_tensor *moved = nullptr;
    if (s->device_type != dst->device_type || s->device_index != dst->device_index) {
        // bring the source to dst's device first, keeping its (broadcast) layout
        if (dst->device_type == GT_DEV_CUDA) {
            moved = gt_to_device_dense(s, dst->device_index, -1);
        } else {
            moved = gt_new_tensor(s->ndim, s->shape, s->dtype, GT_DEV_CPU, 0);
            if (moved) {
                gt_tensor *dd = gt_to_device_dense(s, s->device_index, -1);
                if (!dd || !gt_copy_device_to_host(moved, dd)) {
                    gt_tensor_free(moved);
                    moved = nullptr;
                }
                gt_tensor_free(dd);
            }
        }
        if (!moved) rc = -1;
        s = moved;
    }
    if (rc == 0) {
        if (dst->device_type == GT_DEV_CUDA) {
            rc = device_convert(s, dst) ? 0 : -1;
        } else {
            host_convert(s, dst);
        }
    }
    gt_tensor_free(moved);
    gt_tensor_free(dense_src);
    return rc;
}

extern "C" gt_tensor *gt_tensor_clone(const gt_tensor *t) {
    if (!t) {
        gt_set_error("clone: NULL tensor");
        return nullptr;
    }
    if (t->device_type == GT_DEV_CUDA) return gt_to_device_dense(t, t->device_index, -1);
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, t->dtype, GT_DEV_CPU, 0);
    if (!out) return nullptr;
    if (gt_is_quantized(t->dtype)) {
        std::memcpy(out->storage->ptr, t->storage->ptr, gt_dtype_nbytes(t->dtype, t->numel));
    } else {
        host_convert(t, out);
    }
    return out;
}

extern "C" gt_tensor *gt_tensor_contiguous(const gt_tensor *t) {
    if (!t) {
        gt_set_error("contiguous: NULL tensor");
        return nullptr;
    }
    if (gt_is_quantized(t->dtype) || (gt_is_dense(t) && t->offset == 0)) {
        auto *out = new gt_tensor(*t);  // a view sharing storage
        return out;
    }
    return gt_tensor_clone(t);
}

extern "C" gt_tensor *gt_tensor_to_device(const gt_tensor *t, int device_type, int device_index) {
    if (!t) {
        gt_set_error("to_device: NULL tensor");
        return nullptr;
    }
    if (device_type == GT_DEV_CUDA) return gt_to_device_dense(t, device_index, -1);
    if (device_type != GT_DEV_CPU) {
        gt_set_error("to_device: device type " + std::to_string(device_type) + " is not supported");
        return nullptr;
    }
    if (t->device_type == GT_DEV_CPU) return gt_tensor_clone(t);
    gt_tensor *dense = (gt_is_quantized(t->dtype) || gt_is_dense(t)) ? nullptr : gt_to_device_dense(t, t->device_index, -1);
    const gt_tensor *s = dense ? dense : t;
    if (!gt_is_quantized(t->dtype) && !gt_is_dense(t) && !dense) return nullptr;
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, t->dtype, GT_DEV_CPU, 0);
    if (out && !gt_copy_device_to_host(out, s)) {
        gt_tensor_free(out);
        out = nullptr;
    }
    gt_tensor_free(dense);
    return out;
}

// Float/int conversions (csrc/gt_core.cpp:784-847); quantized targets go through gt_quantize.
extern "C" gt_tensor *gt_tensor_to_dtype(const gt_tensor *t, int dtype) {
    if (!t) {
        gt_set_error("to_dtype: NULL tensor");
        return nullptr;
    }
    if (dtype == GT_Q8_0) return gt_quantize(t, GT_Q8_0 - GT_Q_BASE);
    if (gt_is_quantized(t->dtype)) return gt_dequantize(t, dtype);
    if (t->device_type == GT_DEV_CUDA) return gt_to_device_dense(t, t->device_index, dtype);
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, dtype, GT_DEV_CPU, 0);
    if (out) host_convert(t, out);
    return out;
}

// ---------------------------------------------------------------------------------------------
// DLPack export (unversioned DLManagedTensor ABI, dlpack.h v0.8)
// ---------------------------------------------------------------------------------------------

namespace {
struct DLDevice {
    int32_t device_type;
    int32_t device_id;
};
struct DLDataType {
    uint8_t code;
    uint8_t bits;
    uint16_t lanes;
};
struct DLTensor {
    void *data;
    DLDevice device;
    int32_t ndim;
    DLDataType dtype;
    int64_t *shape;
    int64_t *strides;
    uint64_t byte_offset;
};
struct DLManagedTensor {
    DLTensor dl_tensor;
    void *manager_ctx;
    void (*deleter)(DLManagedTensor *self);
};
struct DLExport {
    DLManagedTensor managed;
    std::shared_ptr<gt_storage> storage;  // keeps the memory alive until torch drops it
    int64_t shape[GT_MAX_DIMS];
    int64_t strides[GT_MAX_DIMS];
};
constexpr int32_t kDLCPU = 1, kDLROCM = 10;
constexpr uint8_t kDLInt = 0, kDLUInt = 1, kDLFloat = 2, kDLBfloat = 4, kDLBool = 6;

void dl_deleter(DLManagedTensor *self) { delete static_cast<DLExport *>(self->manager_ctx); }

bool dl_dtype(int dtype, DLDataType *out) {
    switch (dtype) {
        case GT_F32: *out = {kDLFloat, 32, 1}; return true;
        case GT_F16: *out = {kDLFloat, 16, 1}; return true;
        case GT_BF16: *out = {kDLBfloat, 16, 1}; return true;
        case GT_F64: *out = {kDLFloat, 64, 1}; return true;
        case GT_I8: *out = {kDLInt, 8, 1}; return true;
        case GT_U8: *out = {kDLUInt, 8, 1}; return true;
        case GT_I16: *out = {kDLInt, 16, 1}; return true;
        case GT_I32: *out = {kDLInt, 32, 1}; return true;
        case GT_I64: *out = {kDLInt, 64, 1}; return true;
        case GT_BOOL: *out = {kDLBool, 8, 1}; return true;
        default: return false;
    }
}
}  // namespace

extern "C" void *gt_tensor_to_dlpack(const gt_tensor *t) {
    if (!t || !t->storage) {
        gt_set_error("to_dlpack: NULL tensor");
        return nullptr;
    }
    auto *e = new DLExport();
    e->storage = t->storage;
    DLTensor &d = e->managed.dl_tensor;
    if (gt_is_quantized(t->dtype)) {
        // the raw blocks, as a 1-D uint8 array
        d.dtype = {kDLUInt, 8, 1};
        d.ndim = 1;
        e->shape[0] = (int64_t)gt_dtype_nbytes(t->dtype, t->numel);
        e->strides[0] = 1;
    } else {
        if (!dl_dtype(t->dtype, &d.dtype)) {
            delete e;
            gt_set_error(std::string("to_dlpack: dtype ") + gt_dtype_name(t->dtype) + " has no DLPack code here");
            return nullptr;
        }
        d.ndim = t->ndim;
        for (int i = 0; i < t->ndim; ++i) {
            e->shape[i] = t->shape[i];
            e->strides[i] = t->strides[i];
        }
    }
    // the element offset goes into the pointer (consumers differ in how they treat byte_offset)
    d.byte_offset = 0;
    d.data = gt_data(t);
    d.device = {t->device_type == GT_DEV_CUDA ? kDLROCM : kDLCPU, t->device_type == GT_DEV_CUDA ? t->device_index : 0};
    d.shape = e->shape;
    d.strides = e->strides;
    e->managed.manager_ctx = e;
    e->managed.deleter = dl_deleter;
    return &e->managed;
}
